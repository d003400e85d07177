/*
 * hl_oracle.c — CPU restatement of the reference's attention-stage math.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP kernels:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it.  The product library never links or calls it.
 *
 * Sources restated (monofuel/hippo_leap, paths relative to src/hippo_leap):
 *   tensor.nim:63-81    matmul        i -> j -> p loop, fp32 accumulator
 *   tensor.nim:83-100   rmsnorm       ss sum, inv = 1/sqrt(ss/dim + eps)
 *   tensor.nim:102-118  rmsnormCols   same per column of a col-major tensor
 *   tensor.nim:120-139  softmaxLastDim  max from element 0, exp, sum, *1/sum
 *   tensor.nim:141-166  ropeInplace   interleaved pairs (2i, 2i+1)
 *   tensor.nim:42-54    add / mul     scale and mask glue
 *   quant.nim:78-96     halfToFloat   exact IEEE half decode
 *   quant.nim:98-107    floatToHalf   truncating, flush-to-zero (not used for
 *                                     caches; kept to document the difference)
 * and the semantics tensor.nim leaves to the GPU backend (backends/naive.nim):
 *   :3307-3308, 3400-3401  GQA mapping kvh = h / (Hq/Hkv)
 *   :3328, 3374            score = dot * (1/sqrtf(D)), scale after the dot
 *   :3403                  causal extent j <= i
 *   :3020-3030, 3066-3073  half-split RoPE (i, i+ropeDim/2); dims >= ropeDim pass
 *   :3850-3861             theta table powf(1/base, 2i/ropeDim) in fp32
 *   :3565-3567, 3239       cache layout [kvDim, maxLen], column = position
 *   :4066-4074             qkNorm before RoPE
 *   :1922-2127             argmax (two-pass reduction, its tie order)
 *   :2975-3001             token embedding lookup
 * and GGUF weight rows (quant.nim:235-355: dequantRowQ8_0, Q4K, Q6K).
 *
 * Every routine is single-threaded scalar fp32 code (built -O2, no
 * fast-math), like the reference's CPU path.  fp16/bf16 inputs enter as
 * their stored bits and are upcast exactly.
 *
 * Pinning status (what checks each function; see tests/test_oracle.py):
 *   matmul, softmax, rmsnorm(+Cols), rope (both styles), theta table,
 *   attention decode/prefill: fp64 brute force + closed forms + torch
 *   scaled_dot_product_attention (fp64) through the golden fixtures.
 *   halfToFloat: the reference KAT tests/test_quant.nim:5-15.
 *   argmax: numpy argmax on tie-free inputs, hand-derived tie winners of
 *   the reduction tree, NaN / -inf / all-invalid cases.
 *   embedding: numpy fancy indexing.
 *   GGUF dequant: blocks packed in the tests from the GGUF format's
 *   definition with chosen scales/mins/quants (expected values from the
 *   format formula), including the high-index 6-bit scale packing.
 *   f32->f16/bf16 RNE: numpy / torch conversions (exhaustive over a sweep).
 *   Device transcendental functions of the reference (hippo's expf, powf,
 *   cosf, sinf) are not pinned by any reference test: parity unpinned at
 *   that boundary; tolerance-based only.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_F32 0
#define ORC_F16 1
#define ORC_BF16 2
#define ORC_FP8 3

/* ---------------------------------------------------------------------- */
/* Seeded input generator (shared by tests, fixtures and the CPU baseline) */
/* ---------------------------------------------------------------------- */

static uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

/* uniform in [0,1) with 24 random bits, counter-based on (seed, i) */
static double u01(uint64_t seed, uint64_t i) {
  uint64_t r = splitmix64(seed * 0x100000001B3ull ^ splitmix64(i));
  return (double)(r >> 40) * (1.0 / 16777216.0);
}

void orc_fill_uniform(float* out, int64_t n, uint64_t seed, float lo, float hi) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = (float)(lo + (hi - lo) * u01(seed, (uint64_t)i));
}

/* Box-Muller on counter pairs: element i uses counters (2*(i/2), +1). */
void orc_fill_normal(float* out, int64_t n, uint64_t seed, float mean, float std) {
  for (int64_t i = 0; i < n; ++i) {
    uint64_t c = (uint64_t)(i & ~(int64_t)1);
    double u1 = u01(seed, c) + (1.0 / 33554432.0); /* (0,1] */
    double u2 = u01(seed, c + 1);
    double r = sqrt(-2.0 * log(u1));
    double z = (i & 1) ? r * sin(6.283185307179586 * u2) : r * cos(6.283185307179586 * u2);
    out[i] = (float)(mean + std * z);
  }
}

/* ---------------------------------------------------------------------- */
/* Storage-type conversions                                               */
/* ---------------------------------------------------------------------- */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* quant.nim:78-96 halfToFloat: exact decode, written from its branches. */
float orc_half_to_float(uint16_t h) {
  uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1Fu, f = h & 0x3FFu;
  if (e == 0) {
    if (f == 0) return s ? -0.0f : 0.0f;
    return (s ? -1.0f : 1.0f) * powf(2.0f, -14.0f) * ((float)f / 1024.0f);
  } else if (e == 31) {
    if (f == 0) return s ? -INFINITY : INFINITY;
    return NAN;
  }
  float mant = 1.0f + (float)f / 1024.0f;
  return (s ? -1.0f : 1.0f) * mant * powf(2.0f, (float)((int)e - 15));
}

/* quant.nim:98-107 floatToHalf: truncates the mantissa and flushes |x| <
 * 2^-14 to signed zero.  Documented only; caches use orc_float_to_half_rne. */
uint16_t orc_float_to_half_trunc(float f) {
  uint32_t bits = f2u(f);
  uint16_t s = (uint16_t)((bits >> 16) & 0x8000u);
  int e = (int)((bits >> 23) & 0xFFu) - 127;
  uint32_t m = bits & 0x7FFFFFu;
  if (e <= -15) return s;
  if (e > 15) return s | 0x7C00u;
  return s | (uint16_t)((e + 15) << 10) | (uint16_t)(m >> 13);
}

/* IEEE binary16 round-to-nearest-even with subnormals, inf and NaN. */
uint16_t orc_float_to_half_rne(float f) {
  uint32_t x = f2u(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) /* inf / nan */
    return sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u);
  if (ax >= 0x477FF000u) return sign | 0x7C00u; /* rounds to >= 65520 -> inf */
  if (ax < 0x38800000u) { /* below 2^-14: subnormal or zero */
    /* value = ax as float; half subnormal unit = 2^-24 */
    float a = u2f(ax);
    float scaled = a * 16777216.0f; /* exact: multiply by 2^24 */
    /* round half to even in integer units */
    float r = nearbyintf(scaled);  /* default rounding mode is RNE */
    return sign | (uint16_t)r;
  }
  uint32_t mant = ax & 0x7FFFFFu;
  int e = (int)(ax >> 23) - 127 + 15;
  uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* may carry into exp */
  return sign | (uint16_t)h;
}

float orc_bf16_to_float(uint16_t b) { return u2f((uint32_t)b << 16); }

uint16_t orc_float_to_bf16_rne(float f) {
  uint32_t x = f2u(f);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u); /* quiet NaN */
  uint32_t lsb = (x >> 16) & 1u;
  x += 0x7FFFu + lsb;
  return (uint16_t)(x >> 16);
}

/* OCP fp8 e4m3 ("e4m3fn": bias 7, no infinities, max 448), the library's
 * fp8 KV storage (the reference has no fp8).  Encode: round to nearest even
 * by the value's quantum, saturate at +-448 (infinities too), NaN -> 0x7F
 * with the sign kept.  Written from the format's definition (frexp and a
 * rounding of |x| / quantum), independently of the kernels' bit arithmetic. */
uint8_t orc_float_to_e4m3(float f) {
  const uint8_t sign = signbit(f) ? 0x80 : 0;
  if (isnan(f)) return (uint8_t)(sign | 0x7F);
  const double a = fabs((double)f);
  if (a >= 448.0) return (uint8_t)(sign | 0x7E);
  int e;
  frexp(a, &e);                     /* a in [2^(e-1), 2^e) */
  int ex = e - 1;
  if (ex < -6) ex = -6;             /* below 2^-6 the quantum stays 2^-9 */
  const double q = ldexp(1.0, ex - 3);
  const double r = nearbyint(a / q) * q; /* ties to even (default mode) */
  if (r == 0.0) return sign;
  if (r >= 448.0) return (uint8_t)(sign | 0x7E);
  int e2;
  frexp(r, &e2);
  const int E = e2 - 1;
  if (E < -6) return (uint8_t)(sign | (uint8_t)(r / ldexp(1.0, -9)));
  const int mant = (int)((r / ldexp(1.0, E) - 1.0) * 8.0);
  return (uint8_t)(sign | (uint8_t)(((E + 7) << 3) | mant));
}

float orc_e4m3_to_float(uint8_t b) {
  const int e = (b >> 3) & 15, m = b & 7;
  float v;
  if (e == 15 && m == 7) v = NAN;
  else if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return (b & 0x80) ? -v : v;
}

void orc_convert_from_f32(int dtype, const float* src, void* dst, int64_t n) {
  if (dtype == ORC_F32) { memcpy(dst, src, (size_t)n * 4); return; }
  if (dtype == ORC_FP8) {
    for (int64_t i = 0; i < n; ++i) ((uint8_t*)dst)[i] = orc_float_to_e4m3(src[i]);
    return;
  }
  uint16_t* d = (uint16_t*)dst;
  for (int64_t i = 0; i < n; ++i)
    d[i] = dtype == ORC_F16 ? orc_float_to_half_rne(src[i]) : orc_float_to_bf16_rne(src[i]);
}

void orc_upcast_to_f32(int dtype, const void* src, float* dst, int64_t n) {
  if (dtype == ORC_F32) { memcpy(dst, src, (size_t)n * 4); return; }
  if (dtype == ORC_FP8) {
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_e4m3_to_float(((const uint8_t*)src)[i]);
    return;
  }
  const uint16_t* s = (const uint16_t*)src;
  for (int64_t i = 0; i < n; ++i)
    dst[i] = dtype == ORC_F16 ? orc_half_to_float(s[i]) : orc_bf16_to_float(s[i]);
}

/* ---------------------------------------------------------------------- */
/* tensor.nim restatements                                                */
/* ---------------------------------------------------------------------- */

/* tensor.nim:63-81: c[m,n] = a[m,k] * b[k,n], row-major, loop i, j, p. */
void orc_matmul(const float* a, const float* b, float* c, int m, int k, int n) {
  for (int i = 0; i < m; ++i) {
    const float* arow = a + (int64_t)i * k;
    for (int j = 0; j < n; ++j) {
      float acc = 0.0f;
      for (int p = 0; p < k; ++p) acc += arow[p] * b[(int64_t)p * n + j];
      c[(int64_t)i * n + j] = acc;
    }
  }
}

/* tensor.nim:120-139: softmax over the last dim, written to out. */
void orc_softmax_last_dim(const float* x, float* out, int64_t outer, int dim) {
  for (int64_t o = 0; o < outer; ++o) {
    const float* xr = x + o * dim;
    float* yr = out + o * dim;
    float maxv = xr[0];
    for (int i = 1; i < dim; ++i) maxv = fmaxf(maxv, xr[i]);
    float sum = 0.0f;
    for (int i = 0; i < dim; ++i) {
      float v = expf(xr[i] - maxv);
      yr[i] = v;
      sum += v;
    }
    float inv = 1.0f / sum;
    for (int i = 0; i < dim; ++i) yr[i] *= inv;
  }
}

/* tensor.nim:83-100: RMSNorm of each length-dim row. */
void orc_rmsnorm(const float* x, const float* w, float* out, int64_t outer, int dim, float eps) {
  for (int64_t o = 0; o < outer; ++o) {
    const float* xr = x + o * dim;
    float ss = 0.0f;
    for (int i = 0; i < dim; ++i) ss += xr[i] * xr[i];
    float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = 0; i < dim; ++i) out[o * dim + i] = xr[i] * inv * w[i];
  }
}

/* tensor.nim:102-118: RMSNorm over rows for each column of [dim, seq]. */
void orc_rmsnorm_cols(const float* x, const float* w, float* out, int dim, int seq, float eps) {
  for (int s = 0; s < seq; ++s) {
    float ss = 0.0f;
    for (int r = 0; r < dim; ++r) { float v = x[(int64_t)r * seq + s]; ss += v * v; }
    float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int r = 0; r < dim; ++r)
      out[(int64_t)r * seq + s] = x[(int64_t)r * seq + s] * inv * w[r];
  }
}

/* tensor.nim:141-166: interleaved RoPE on [outer, seq, dim] row-major. */
void orc_rope_inplace(float* x, int64_t outer, int seq, int dim, float base, int start_pos) {
  float inv_base = 1.0f / base;
  for (int64_t o = 0; o < outer; ++o)
    for (int p = 0; p < seq; ++p) {
      float pos = (float)(start_pos + p);
      float* row = x + (o * seq + p) * dim;
      for (int i = 0; i < dim / 2; ++i) {
        float theta = powf(inv_base, (float)(2 * i) / (float)dim);
        float angle = pos * theta;
        float c = cosf(angle), s = sinf(angle);
        float v0 = row[2 * i], v1 = row[2 * i + 1];
        row[2 * i] = v0 * c - v1 * s;
        row[2 * i + 1] = v0 * s + v1 * c;
      }
    }
}

/* ---------------------------------------------------------------------- */
/* naive.nim semantics                                                    */
/* ---------------------------------------------------------------------- */

/* naive.nim:3850-3861: theta[i] = pow(1/base, 2i/ropeDim), fp32. */
void orc_rope_theta_table(float* theta, int rope_dim, float base) {
  for (int i = 0; i < rope_dim / 2; ++i)
    theta[i] = powf(1.0f / base, (2.0f * (float)i) / (float)rope_dim);
}

/* One head vector x[head_dim] (stride `stride` between dims) rotated at
 * `pos`.  style 0: half-split pairs (i, i+rope_dim/2) (naive.nim:3066-3073);
 * style 1: interleaved (2i, 2i+1) (tensor.nim:156-166).  Dims >= rope_dim
 * are untouched (naive.nim:3200-3201).  angle = float(pos) * theta[i].   */
static void rope_vec(float* x, int64_t stride, int rope_dim, const float* theta, int pos, int style) {
  int half = rope_dim / 2;
  for (int i = 0; i < half; ++i) {
    float angle = (float)pos * theta[i];
    float c = cosf(angle), s = sinf(angle);
    int64_t i0 = style == 0 ? i : 2 * i;
    int64_t i1 = style == 0 ? i + half : 2 * i + 1;
    float v0 = x[i0 * stride], v1 = x[i1 * stride];
    x[i0 * stride] = v0 * c - v1 * s;
    x[i1 * stride] = v0 * s + v1 * c;
  }
}

/* Decode-side RoPE of x[n_head*head_dim] at pos (ropeQKDecodeKernel,
 * naive.nim:3046-3073, for one of q / k). */
void orc_rope_heads(float* x, int n_head, int head_dim, int rope_dim, const float* theta,
                    int pos, int style) {
  for (int h = 0; h < n_head; ++h) rope_vec(x + (int64_t)h * head_dim, 1, rope_dim, theta, pos, style);
}

/* Prefill-side RoPE of col-major x[n_head*head_dim, seq]: column p at
 * position pos0 + p (ropeAtPosThetaKernel naive.nim:3116-3131; with pos0 = 0
 * this is ropeAtPosKernel's prefill branch naive.nim:3031-3044). */
void orc_rope_cols(float* x, int n_head, int head_dim, int seq, int rope_dim, const float* theta,
                   int pos0, int style) {
  for (int h = 0; h < n_head; ++h)
    for (int p = 0; p < seq; ++p)
      rope_vec(x + (int64_t)h * head_dim * seq + p, seq, rope_dim, theta, pos0 + p, style);
}

/* qkNormKernel (naive.nim:2887-2916): per-head RMSNorm in place; the
 * formula is tensor.nim:92-100's. */
void orc_qk_norm(float* x, const float* w, int n_head, int head_dim, float eps) {
  orc_rmsnorm(x, w, x, n_head, head_dim, eps);
}

/* qkNormPrefillKernel (naive.nim:2928-2960): per (head, column) on
 * col-major [n_head*head_dim, seq]. */
void orc_qk_norm_cols(float* x, const float* w, int n_head, int head_dim, int seq, float eps) {
  for (int h = 0; h < n_head; ++h) {
    float* xh = x + (int64_t)h * head_dim * seq;
    orc_rmsnorm_cols(xh, w, xh, head_dim, seq, eps);
  }
}

/* storeKVKernel (naive.nim:3228-3239): cache[r*cols + start + c] = src[r*src_cols + c],
 * written in the cache dtype with RNE. */
void orc_store_kv(void* cache, int dtype, const float* src, int rows, int src_cols, int cache_cols,
                  int start_pos) {
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < src_cols; ++c) {
      int64_t di = (int64_t)r * cache_cols + start_pos + c;
      float v = src[(int64_t)r * src_cols + c];
      if (dtype == ORC_F32) ((float*)cache)[di] = v;
      else if (dtype == ORC_F16) ((uint16_t*)cache)[di] = orc_float_to_half_rne(v);
      else ((uint16_t*)cache)[di] = orc_float_to_bf16_rne(v);
    }
}

/* Decode attention (attentionDecodeKernel's math, naive.nim:3292-3367,
 * composed from tensor.nim ops): for each query head h,
 *   scores[1,L] = matmul(q_h[1,D], K_kvh[D,L]) * scale      (tensor.nim:63-81, 49-54)
 *   p = softmaxLastDim(scores)                              (tensor.nim:120-139)
 *   o_h[1,D] = matmul(p[1,L], V_kvh^T[L,D])
 * K_kvh / V_kvh are rows kvh*D .. kvh*D+D-1 of the fp32 caches
 * [Hkv*D, max_len], columns 0..L-1.  `scores` is caller scratch [L]. */
void orc_attention_decode(const float* q, const float* kc, const float* vc, float* out, int n_head,
                          int n_head_kv, int head_dim, int L, int max_len, float scale,
                          float* scores) {
  int group = n_head / n_head_kv;
  for (int h = 0; h < n_head; ++h) {
    int kvh = h / group;
    const float* qh = q + (int64_t)h * head_dim;
    const float* K = kc + (int64_t)kvh * head_dim * max_len;
    const float* V = vc + (int64_t)kvh * head_dim * max_len;
    for (int j = 0; j < L; ++j) {
      float acc = 0.0f;
      for (int p = 0; p < head_dim; ++p) acc += qh[p] * K[(int64_t)p * max_len + j];
      scores[j] = acc * scale;
    }
    orc_softmax_last_dim(scores, scores, 1, L);
    for (int d = 0; d < head_dim; ++d) {
      float acc = 0.0f;
      for (int p = 0; p < L; ++p) acc += scores[p] * V[(int64_t)d * max_len + p];
      out[(int64_t)h * head_dim + d] = acc;
    }
  }
}

/* Causal prefill attention (attentionPrefillKernel's math, naive.nim:3385-3447)
 * over col-major Q[Hq*D, T], K/V[Hkv*D, T]; O col-major [Hq*D, T].  Row i of
 * head h attends to j <= i.  Only heads [h0,h1) and rows r0, r0+rstep, ... < r1
 * are written, so a test can check sampled rows of a large case.  `scores`
 * is caller scratch [T]. */
void orc_attention_prefill(const float* Q, const float* K, const float* V, float* O, int n_head,
                           int n_head_kv, int head_dim, int T, float scale, int h0, int h1,
                           int r0, int r1, int rstep, float* scores) {
  int group = n_head / n_head_kv;
  for (int h = h0; h < h1; ++h) {
    int kvh = h / group;
    const float* Qh = Q + (int64_t)h * head_dim * T;
    const float* Kh = K + (int64_t)kvh * head_dim * T;
    const float* Vh = V + (int64_t)kvh * head_dim * T;
    for (int i = r0; i < r1; i += rstep) {
      int n = i + 1;
      for (int j = 0; j < n; ++j) {
        float acc = 0.0f;
        for (int p = 0; p < head_dim; ++p) acc += Qh[(int64_t)p * T + i] * Kh[(int64_t)p * T + j];
        scores[j] = acc * scale;
      }
      orc_softmax_last_dim(scores, scores, 1, n);
      for (int d = 0; d < head_dim; ++d) {
        float acc = 0.0f;
        for (int p = 0; p < n; ++p) acc += scores[p] * Vh[(int64_t)d * T + p];
        O[((int64_t)h * head_dim + d) * T + i] = acc;
      }
    }
  }
}

/* tensor.nim add (:42-47): out[i] = a[i] + b[i] (fp32). */
void orc_add(const float* a, const float* b, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* gpuSiluMul's kernel (siluMulKernel, naive.nim:2179-2187): with x = gate[i],
 * out[i] = x * (1 / (1 + expf(-x))) * up[i], in that order (the CPU
 * tensor.nim silu, :56-61, writes x / (1 + exp(-x)); the GPU form is the
 * one the drop-in replaces). */
void orc_silu_mul(const float* gate, const float* up, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float x = gate[i];
    const float sig = 1.0f / (1.0f + expf(-x));
    out[i] = x * sig * up[i];
  }
}

/* ---------------------------------------------------------------------- */
/* Decode-step ends (backends/naive.nim)                                  */
/* ---------------------------------------------------------------------- */

/* One 256-thread block reduction of argmaxPass1Kernel / argmaxPass2Kernel
 * (naive.nim:1942-1977, 2009-2044) on (val[256], idx[256]): the LDS steps
 * 128 and 64, then wave64 shuffle-downs 32..1, each replacing only on a
 * strictly greater value; lanes whose source is past lane 63 keep their own
 * value (shuffle-down semantics).  Returns lane 0's (value, index). */
static void orc_argmax_block(float* sv, int* si, float* out_v, int* out_i) {
  for (int t = 0; t < 128; ++t)
    if (sv[t + 128] > sv[t]) { sv[t] = sv[t + 128]; si[t] = si[t + 128]; }
  for (int t = 0; t < 64; ++t)
    if (sv[t + 64] > sv[t]) { sv[t] = sv[t + 64]; si[t] = si[t + 64]; }
  for (int off = 32; off >= 1; off >>= 1) {
    float nv[64];
    int ni[64];
    for (int l = 0; l < 64; ++l) {
      float ov = l + off < 64 ? sv[l + off] : sv[l];
      int oi = l + off < 64 ? si[l + off] : si[l];
      nv[l] = sv[l];
      ni[l] = si[l];
      if (ov > nv[l]) { nv[l] = ov; ni[l] = oi; }
    }
    memcpy(sv, nv, sizeof(nv));
    memcpy(si, ni, sizeof(ni));
  }
  *out_v = sv[0];
  *out_i = si[0];
}

/* gpuArgmax (naive.nim:2105-2127) with the reference's geometry
 * (ArgmaxGridBlocks = 256 blocks of 256 threads, naive.nim:2092):
 * pass 1 (naive.nim:1922-1977): thread (b, t) scans i = b*256 + t, then
 * i += 65536, keeping the first strictly greater value from -3.4e38 and
 * index -1; each block reduces to (value, index).  Pass 2
 * (naive.nim:1999-2044): one block reduces the 256 block results. */
int orc_argmax(const float* x, int64_t n) {
  static float bv[256], sv[256];
  static int bi[256], si[256];
  for (int b = 0; b < 256; ++b) {
    for (int t = 0; t < 256; ++t) {
      float v = -3.4e38f;
      int idx = -1;
      for (int64_t i = (int64_t)b * 256 + t; i < n; i += 65536)
        if (x[i] > v) { v = x[i]; idx = (int)i; }
      sv[t] = v;
      si[t] = idx;
    }
    orc_argmax_block(sv, si, &bv[b], &bi[b]);
  }
  float v;
  int idx;
  orc_argmax_block(bv, bi, &v, &idx);
  return idx;
}

/* gpuEmbedding (naive.nim:2975-3001): out[e*nTokens + t] =
 * w[tok[t]*nEmb + e]; fp32 copy, token ids assumed in range. */
void orc_embedding(const float* w, const int* tok, float* out, int n_emb, int n_tokens) {
  for (int e = 0; e < n_emb; ++e)
    for (int t = 0; t < n_tokens; ++t)
      out[(int64_t)e * n_tokens + t] = w[(int64_t)tok[t] * n_emb + e];
}

/* ---------------------------------------------------------------------- */
/* GGUF weight rows (quant.nim)                                           */
/* ---------------------------------------------------------------------- */

static float orc_half_at(const uint8_t* p) { return orc_half_to_float((uint16_t)(p[0] | (p[1] << 8))); }

/* quant.nim:304-319: 34-byte blocks, fp16 d then 32 int8; x = q * d. */
static void orc_dequant_q8_0(const uint8_t* src, float* dst, int k) {
  for (int b = 0; b < k / 32; ++b) {
    const uint8_t* blk = src + (int64_t)b * 34;
    const float d = orc_half_at(blk);
    for (int j = 0; j < 32; ++j) dst[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
  }
}

/* quant.nim:235-242 (getScaleMinK4): 6-bit scale / min j of the 12 bytes. */
static void orc_scale_min_k4(int j, const uint8_t* s, int* sc, int* mn) {
  if (j < 4) {
    *sc = s[j] & 63;
    *mn = s[j + 4] & 63;
  } else {
    *sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
    *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

/* quant.nim:244-277: 144-byte blocks of 256: d, dmin, 12 scale bytes, 128
 * nibble bytes; each 64-element chunk uses 32 bytes, low nibbles first. */
static void orc_dequant_q4k(const uint8_t* src, float* dst, int k) {
  for (int b = 0; b < k / 256; ++b) {
    const uint8_t* blk = src + (int64_t)b * 144;
    const float d = orc_half_at(blk), dmin = orc_half_at(blk + 2);
    const uint8_t* scales = blk + 4;
    const uint8_t* q = blk + 16;
    float* out = dst + b * 256;
    for (int c = 0; c < 4; ++c) {
      int sc, mn;
      orc_scale_min_k4(2 * c, scales, &sc, &mn);
      const float d1 = d * (float)sc, m1 = dmin * (float)mn;
      orc_scale_min_k4(2 * c + 1, scales, &sc, &mn);
      const float d2 = d * (float)sc, m2 = dmin * (float)mn;
      for (int l = 0; l < 32; ++l) out[64 * c + l] = d1 * (float)(q[32 * c + l] & 0x0F) - m1;
      for (int l = 0; l < 32; ++l) out[64 * c + 32 + l] = d2 * (float)(q[32 * c + l] >> 4) - m2;
    }
  }
}

/* quant.nim:321-355: 210-byte blocks of 256: ql[128], qh[64], int8 sc[16],
 * fp16 d; two halves of 128 elements, four 32-element groups each. */
static void orc_dequant_q6k(const uint8_t* src, float* dst, int k) {
  for (int b = 0; b < k / 256; ++b) {
    const uint8_t* blk = src + (int64_t)b * 210;
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    const float d = orc_half_at(blk + 208);
    float* out = dst + b * 256;
    for (int n = 0; n < 2; ++n) {
      for (int l = 0; l < 32; ++l) {
        const int is = l / 16;
        const int q1 = (int)((ql[64 * n + l] & 0xF) | (((qh[32 * n + l] >> 0) & 3) << 4)) - 32;
        const int q2 = (int)((ql[64 * n + l + 32] & 0xF) | (((qh[32 * n + l] >> 2) & 3) << 4)) - 32;
        const int q3 = (int)((ql[64 * n + l] >> 4) | (((qh[32 * n + l] >> 4) & 3) << 4)) - 32;
        const int q4 = (int)((ql[64 * n + l + 32] >> 4) | (((qh[32 * n + l] >> 6) & 3) << 4)) - 32;
        out[128 * n + l] = d * (float)sc[8 * n + is + 0] * (float)q1;
        out[128 * n + l + 32] = d * (float)sc[8 * n + is + 2] * (float)q2;
        out[128 * n + l + 64] = d * (float)sc[8 * n + is + 4] * (float)q3;
        out[128 * n + l + 96] = d * (float)sc[8 * n + is + 6] * (float)q4;
      }
    }
  }
}

/* quant.nim:132-170: 84-byte blocks of 256: 16 scale bytes (low nibble
 * scale, high nibble min), 64 bytes of 2-bit quants, fp16 d, fp16 dmin.
 * Element 128n + 32j + 16g + l: bits 2j of qs[32n + 16g + l], scale byte
 * 8n + 2j + g. */
static void orc_dequant_q2k(const uint8_t* src, float* dst, int k) {
  for (int b = 0; b < k / 256; ++b) {
    const uint8_t* blk = src + (int64_t)b * 84;
    const uint8_t* sc = blk;
    const uint8_t* qs = blk + 16;
    const float d = orc_half_at(blk + 80), dmin = orc_half_at(blk + 82);
    float* out = dst + b * 256;
    for (int n = 0; n < 2; ++n)
      for (int j = 0; j < 4; ++j)
        for (int g = 0; g < 2; ++g) {
          const int s = sc[8 * n + 2 * j + g];
          const float dl = d * (float)(s & 0x0F), ml = dmin * (float)(s >> 4);
          for (int l = 0; l < 16; ++l)
            out[128 * n + 32 * j + 16 * g + l] =
                dl * (float)((qs[32 * n + 16 * g + l] >> (2 * j)) & 3) - ml;
        }
  }
}

/* quant.nim:172-233: 110-byte blocks of 256: hmask[32], qs[64], 12 bytes of
 * 6-bit scales, fp16 d.  Element 128n + 32j + 16g + l: bits 2j of
 * qs[32n + 16g + l], minus 4 unless bit 4n + j of hmask[16g + l] is set;
 * scale 8n + 2j + g (6 bits, minus 32). */
static void orc_dequant_q3k(const uint8_t* src, float* dst, int k) {
  for (int b = 0; b < k / 256; ++b) {
    const uint8_t* blk = src + (int64_t)b * 110;
    const uint8_t* hm = blk;
    const uint8_t* qs = blk + 32;
    const uint8_t* s = blk + 96;
    const float d = orc_half_at(blk + 108);
    int scales[16];
    for (int i = 0; i < 16; ++i) {
      const int lo = i < 8 ? (s[i] & 0x0F) : (s[i - 8] >> 4);
      const int hi = (s[8 + (i & 3)] >> (2 * (i >> 2))) & 3;
      scales[i] = (lo | (hi << 4)) - 32;
    }
    float* out = dst + b * 256;
    for (int n = 0; n < 2; ++n)
      for (int j = 0; j < 4; ++j)
        for (int g = 0; g < 2; ++g) {
          const float dl = d * (float)scales[8 * n + 2 * j + g];
          for (int l = 0; l < 16; ++l) {
            const int q = (qs[32 * n + 16 * g + l] >> (2 * j)) & 3;
            const int h = (hm[16 * g + l] >> (4 * n + j)) & 1 ? 0 : 4;
            out[128 * n + 32 * j + 16 * g + l] = dl * (float)(q - h);
          }
        }
  }
}

/* quant.nim:279-302: 22-byte blocks of 32: fp16 d, 32 high bits, 16 nibble
 * bytes; element j < 16 = low nibble of qs[j], j >= 16 = high nibble of
 * qs[j - 16], high bit j; value d * (q - 16). */
static void orc_dequant_q5_0(const uint8_t* src, float* dst, int k) {
  for (int b = 0; b < k / 32; ++b) {
    const uint8_t* blk = src + (int64_t)b * 22;
    const float d = orc_half_at(blk);
    const uint32_t qh = blk[2] | (blk[3] << 8) | (blk[4] << 16) | ((uint32_t)blk[5] << 24);
    for (int j = 0; j < 32; ++j) {
      const int lo = j < 16 ? (blk[6 + j] & 0x0F) : (blk[6 + j - 16] >> 4);
      const int q = lo | (int)(((qh >> j) & 1) << 4);
      dst[b * 32 + j] = d * (float)(q - 16);
    }
  }
}

/* quant.nim:357-383: 24-byte blocks of 32: fp16 d, fp16 m, 32 high bits,
 * 16 nibble bytes (as Q5_0); value d * q + m. */
static void orc_dequant_q5_1(const uint8_t* src, float* dst, int k) {
  for (int b = 0; b < k / 32; ++b) {
    const uint8_t* blk = src + (int64_t)b * 24;
    const float d = orc_half_at(blk), m = orc_half_at(blk + 2);
    const uint32_t qh = blk[4] | (blk[5] << 8) | (blk[6] << 16) | ((uint32_t)blk[7] << 24);
    for (int j = 0; j < 32; ++j) {
      const int lo = j < 16 ? (blk[8 + j] & 0x0F) : (blk[8 + j - 16] >> 4);
      const int q = lo | (int)(((qh >> j) & 1) << 4);
      dst[b * 32 + j] = d * (float)q + m;
    }
  }
}

/* 176-byte blocks of 256: d, dmin, 12 scale bytes (as Q4_K), qh[32],
 * qs[128].  Element 32s + l (sub-block s): nibble s & 1 of qs[32(s/2) + l]
 * plus bit s of qh[l] as bit 4.  This is the GPU kernel's reading
 * (backends/naive.nim:1267-1323), the one hl_gpu_linear_col_quant replaces;
 * quant.nim:385-423 (dequantRowQ5K, CPU side) reads bits (s/2 rounded to
 * even)/2 + s%2 and moves to qs for s >= 4 instead, which differs for s >= 2. */
static void orc_dequant_q5k(const uint8_t* src, float* dst, int k) {
  for (int b = 0; b < k / 256; ++b) {
    const uint8_t* blk = src + (int64_t)b * 176;
    const float d = orc_half_at(blk), dmin = orc_half_at(blk + 2);
    const uint8_t* qh = blk + 16;
    const uint8_t* qs = blk + 48;
    float* out = dst + b * 256;
    for (int s = 0; s < 8; ++s) {
      int sc, mn;
      orc_scale_min_k4(s, blk + 4, &sc, &mn);
      const float dl = d * (float)sc, ml = dmin * (float)mn;
      for (int l = 0; l < 32; ++l) {
        const int nib = (s & 1) ? (qs[32 * (s / 2) + l] >> 4) : (qs[32 * (s / 2) + l] & 0x0F);
        const int q = nib | (((qh[l] >> s) & 1) << 4);
        out[32 * s + l] = dl * (float)q - ml;
      }
    }
  }
}

/* quant.nim:16-17 (kvaluesIQ4NL), 425-441: 18-byte blocks of 32: fp16 d,
 * 16 nibble bytes (as Q5_0) indexing a fixed non-linear table. */
static const int8_t kOrcIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                     1,    13,   25,  38,  53,  69,  89,  113};
static void orc_dequant_iq4nl(const uint8_t* src, float* dst, int k) {
  for (int b = 0; b < k / 32; ++b) {
    const uint8_t* blk = src + (int64_t)b * 18;
    const float d = orc_half_at(blk);
    for (int j = 0; j < 16; ++j) {
      dst[b * 32 + j] = d * (float)kOrcIq4nl[blk[2 + j] & 0x0F];
      dst[b * 32 + j + 16] = d * (float)kOrcIq4nl[blk[2 + j] >> 4];
    }
  }
}

/* Bytes per row of k elements of GGUF type qtype, 0 if not covered. */
int64_t orc_quant_row_bytes(int qtype, int k) {
  switch (qtype) {
    case 1: return 2LL * k;
    case 6: return (int64_t)(k / 32) * 22;
    case 7: return (int64_t)(k / 32) * 24;
    case 8: return (int64_t)(k / 32) * 34;
    case 10: return (int64_t)(k / 256) * 84;
    case 11: return (int64_t)(k / 256) * 110;
    case 12: return (int64_t)(k / 256) * 144;
    case 13: return (int64_t)(k / 256) * 176;
    case 14: return (int64_t)(k / 256) * 210;
    case 20: return (int64_t)(k / 32) * 18;
    default: return 0;
  }
}

/* Rows of GGUF type qtype (1 F16, 6 Q5_0, 7 Q5_1, 8 Q8_0, 10 Q2_K, 11 Q3_K,
 * 12 Q4_K, 13 Q5_K, 14 Q6_K, 20 IQ4_NL) -> fp32 [rows][k]; returns the
 * bytes per row (0: type not covered). */
int64_t orc_dequant_rows(int qtype, const uint8_t* src, float* dst, int rows, int k) {
  const int64_t rb = orc_quant_row_bytes(qtype, k);
  for (int r = 0; r < rows && rb; ++r) {
    const uint8_t* s = src + r * rb;
    float* o = dst + (int64_t)r * k;
    switch (qtype) {
      case 1: for (int i = 0; i < k; ++i) o[i] = orc_half_at(s + 2 * i); break;
      case 6: orc_dequant_q5_0(s, o, k); break;
      case 7: orc_dequant_q5_1(s, o, k); break;
      case 8: orc_dequant_q8_0(s, o, k); break;
      case 10: orc_dequant_q2k(s, o, k); break;
      case 11: orc_dequant_q3k(s, o, k); break;
      case 12: orc_dequant_q4k(s, o, k); break;
      case 13: orc_dequant_q5k(s, o, k); break;
      case 14: orc_dequant_q6k(s, o, k); break;
      case 20: orc_dequant_iq4nl(s, o, k); break;
    }
  }
  return rb;
}
