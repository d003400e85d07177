// Split-K GQA decode attention for gfx950.
//
// Semantics: attentionDecodeKernel / gpuAttentionDecode (backends/naive.nim:
// 3292-3383): o_h = softmax(q_h . K_kvh^T * scale) . V_kvh over cache columns
// [0, L), kvh = h / (Hq/Hkv), caches [Hkv*D, max_len] with the position
// fastest.  The reference runs one 256-thread block per QUERY head and
// re-reads K/V once per head of the group; here one workgroup serves one
// (sequence, kv head, context split) and all G query heads of that kv head, so
// every K/V byte is read once.
//
// Work split: grid = (num_splits, Hkv * head_chunks, B), 256 threads = 4
// waves.  The split's columns are dealt to the waves in 32- (MFMA path) or
// 64-column (fp32 path) tiles; each wave keeps its own online-softmax state
// (running max m, sum l, accumulators o) in registers, the four waves merge
// through LDS, and the workgroup writes one partial (m, l, o[D]) per query
// head.  decode_merge_kernel folds the partials of all splits.
//
// Softmax runs in base 2: q is pre-multiplied by scale*log2(e), so
// p = exp2(s - m) equals the reference's expf(score - max).
#include "common.h"
#include "launch.h"

namespace hl {

// Partial layout in the workspace: for (b, hq, split):
//   ws_o [((b*Hq + hq)*S + split)*D + d]   unnormalised sum p*v
//   ws_ml[((b*Hq + hq)*S + split)*2 + {0,1}]  running max (log2 units), sum
struct DecodeParams {
  const float* q;
  const void* k;
  const void* v;
  float* out;      // final output when direct != 0
  float* ws_o;
  float* ws_ml;
  const int* seq_lens;
  long long batch_stride;
  int n_head, n_head_kv, head_dim, group, head_chunk, n_chunks;
  int max_len, seq_len, split_len, num_splits;
  int direct;      // 1: num_splits == 1, normalise and write out directly
  float scale_log2;
};

// ---------------------------------------------------------------------------
// Workgroup epilogue shared by both kernels: merge the 4 waves' states held
// in LDS and write the split's partial (or the final output).
//   sm_m[w][h], sm_l[w][h], sm_o[w][h][D] for h < hc (heads of this chunk).
// ---------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ void merge_waves_and_store(const DecodeParams& p, const float* sm_m,
                                                      const float* sm_l, const float* sm_o,
                                                      int hc, int b, int hq0, int split,
                                                      int hstride) {
  const int tid = threadIdx.x;
  for (int idx = tid; idx < hc * D; idx += 256) {
    const int h = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sm_m[w * hstride + h]);
    float o = 0.f, l = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = fast_exp2(sm_m[w * hstride + h] - M);
        o += f * sm_o[(w * hstride + h) * D + d];
        l += f * sm_l[w * hstride + h];
      }
    }
    const int hq = hq0 + h;
    const long long row = (long long)b * p.n_head + hq;
    if (p.direct) {
      p.out[row * D + d] = o / l;
    } else {
      const long long pi = row * p.num_splits + split;
      p.ws_o[pi * D + d] = o;
      if (d == 0) {
        p.ws_ml[pi * 2 + 0] = M;
        p.ws_ml[pi * 2 + 1] = l;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 KV path (vector ALU).  A wave owns 64 consecutive columns per tile,
// lane j scores column t0+j for every head of the chunk, then lanes switch to
// owning output dims for the P.V product.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void decode_f32_kernel(DecodeParams p) {
  constexpr int HC = 16;  // max heads per chunk
  constexpr int DPL = (D + 63) / 64;  // output dims per lane
  __shared__ __attribute__((aligned(16))) float sq[HC * D];
  __shared__ float sp[4][HC][64];
  __shared__ float sm_m[4 * HC], sm_l[4 * HC];
  __shared__ float sm_o[4 * HC * D];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int b = blockIdx.z;
  const int kvh = blockIdx.y / p.n_chunks, chunk = blockIdx.y % p.n_chunks;
  const int hq0 = kvh * p.group + chunk * p.head_chunk;
  const int hc = min(p.head_chunk, p.group - chunk * p.head_chunk);
  const int split = blockIdx.x;
  const int L = p.seq_lens ? p.seq_lens[b] : p.seq_len;
  const int s0 = split * p.split_len;
  const int s1 = min(L, s0 + p.split_len);

  const float* qb = p.q + ((long long)b * p.n_head + hq0) * D;
  for (int i = tid; i < HC * D; i += 256) {
    const int h = i / D;
    sq[i] = h < hc ? qb[i] : 0.f;
  }
  __syncthreads();

  const long long base = (long long)b * p.batch_stride + (long long)kvh * D * p.max_len;
  const float* K = (const float*)p.k + base;
  const float* V = (const float*)p.v + base;

  float m_run[HC], l_run[HC], acc[HC][DPL];
#pragma unroll
  for (int h = 0; h < HC; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[h][i] = 0.f;
  }

  for (int t0 = s0 + wave * 64; t0 < s1; t0 += 256) {
    const int col = t0 + lane;
    const bool valid = col < s1;
    float s[HC];
#pragma unroll
    for (int h = 0; h < HC; ++h) s[h] = 0.f;
    if (valid) {
      for (int d = 0; d < D; d += 4) {
        float kv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) kv[u] = K[(long long)(d + u) * p.max_len + col];
#pragma unroll
        for (int h = 0; h < HC; ++h) {
          const f32x4 qv = *(const f32x4*)&sq[h * D + d];
#pragma unroll
          for (int u = 0; u < 4; ++u) s[h] = fmaf(qv[u], kv[u], s[h]);
        }
      }
    }
    // score = dot * scale (naive.nim:3328), here in log2 units
#pragma unroll
    for (int h = 0; h < HC; ++h) s[h] *= p.scale_log2;
    float alpha[HC];
#pragma unroll
    for (int h = 0; h < HC; ++h) {
      if (h < hc) {
        const float sv = valid ? s[h] : -INFINITY;
        const float mt = wave_max(sv);
        const float mn = fmaxf(m_run[h], mt);
        alpha[h] = fast_exp2(m_run[h] - mn);
        const float pv = fast_exp2(sv - mn);
        m_run[h] = mn;
        l_run[h] = l_run[h] * alpha[h] + pv;  // per-lane partial, summed at the end
        sp[wave][h][lane] = pv;
      } else {
        alpha[h] = 1.f;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int nj = min(64, s1 - t0);
#pragma unroll
    for (int h = 0; h < HC; ++h)
#pragma unroll
      for (int i = 0; i < DPL; ++i) acc[h][i] *= alpha[h];
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      const int d = lane + 64 * i;
      if (d < D) {
        const float* vrow = V + (long long)d * p.max_len + t0;
        for (int j = 0; j < nj; ++j) {
          const float vv = vrow[j];
#pragma unroll
          for (int h = 0; h < HC; ++h) acc[h][i] = fmaf(sp[wave][h][j], vv, acc[h][i]);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

#pragma unroll
  for (int h = 0; h < HC; ++h) {
    const float l = wave_sum(l_run[h]);
    if (lane == 0 && h < hc) {
      sm_m[wave * HC + h] = m_run[h];
      sm_l[wave * HC + h] = l;
    }
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      const int d = lane + 64 * i;
      if (d < D && h < hc) sm_o[(wave * HC + h) * D + d] = acc[h][i];
    }
  }
  __syncthreads();
  merge_waves_and_store<D>(p, sm_m, sm_l, sm_o, hc, b, hq0, split, HC);
}

// ---------------------------------------------------------------------------
// fp16 / bf16 KV path on MFMA (v_mfma_f32_16x16x32_{f16,bf16}).
//
// Per 32-column tile a wave computes S^T[col][head] = K^T . Q^T with the 16
// MFMA rows = columns, 16 MFMA cols = heads of the chunk (zero-padded), then
// O[head][d] += P[head][col] . V^T[col][d].  The MFMA output layout of the
// first product (lane = 16*g + c holds rows 4g..4g+3 of column c) is exactly
// the A-operand layout of the second (lane holds 8 k-values of row c), so P
// never leaves registers.  Tile rows are assigned to columns so that the 8
// k-values of lane group g are the 8 consecutive columns t0+8g..t0+8g+7: the
// V operand is then one 16-byte load of a cache row.
//
// K^T fragments need 8 consecutive head dims of one column, which are
// max_len elements apart in the cache: K is staged through LDS (coalesced
// 16-byte global loads, row-major) and gathered with 16-bit LDS reads.
//
// Accuracy: q (fp32) and p (fp32) are split into hi + lo parts of the KV
// storage type and both parts go through the MFMA (the KV values are exact in
// that type), so scores and P.V carry ~16 significant bits per product
// instead of 8 and accumulate in fp32.
// ---------------------------------------------------------------------------
template <int DT>
struct MfmaT;
template <>
struct MfmaT<HL_F16> {
  typedef f16x8 vec;
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct MfmaT<HL_BF16> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <int DT>
__device__ __forceinline__ void split_hi_lo(const float* x, typename MfmaT<DT>::vec& hi,
                                            typename MfmaT<DT>::vec& lo) {
  u16x8 h, l;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint16_t hb = to_bits<DT>(x[e]);
    h[e] = hb;
    l[e] = to_bits<DT>(x[e] - from_bits<DT>(hb));
  }
  hi = __builtin_bit_cast(typename MfmaT<DT>::vec, h);
  lo = __builtin_bit_cast(typename MfmaT<DT>::vec, l);
}

// Loads 8 consecutive 16-bit cache elements [col, col+8) of one row; columns
// >= lim read as zero.  VEC: the 8 elements are 16-byte aligned.
template <bool VEC>
__device__ __forceinline__ u16x8 load_row8(const uint16_t* row, int col, int lim) {
  u16x8 r;
  if (VEC && col + 8 <= lim) {
    r = *(const u16x8*)(row + col);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (col + e < lim) ? row[col + e] : (uint16_t)0;
  }
  return r;
}

template <int D, int DT, bool VEC>
__global__ __launch_bounds__(256, 2) void decode_mfma_kernel(DecodeParams p) {
  typedef typename MfmaT<DT>::vec vec;
  constexpr int KS = D / 32;      // k-steps of the QK^T product
  constexpr int NB = D / 16;      // 16-dim output blocks
  constexpr int PITCH = 40;       // LDS row pitch (elements) of a 32-column K tile
  constexpr int HS = 16;          // head slots of the merge buffers
  constexpr int KT_ELEMS = 4 * D * PITCH;              // 4 wave tiles (uint16)
  constexpr int MERGE_FLOATS = 4 * HS * (D + 2);
  constexpr int LDS_BYTES = (KT_ELEMS * 2 > MERGE_FLOATS * 4) ? KT_ELEMS * 2 : MERGE_FLOATS * 4;
  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[LDS_BYTES];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  const int b = blockIdx.z;
  const int kvh = blockIdx.y / p.n_chunks, chunk = blockIdx.y % p.n_chunks;
  const int hq0 = kvh * p.group + chunk * p.head_chunk;
  const int hc = min(p.head_chunk, p.group - chunk * p.head_chunk);
  const int split = blockIdx.x;
  const int L = p.seq_lens ? p.seq_lens[b] : p.seq_len;
  const int s0 = split * p.split_len;
  const int s1 = min(L, s0 + p.split_len);

  // Q^T operand: lane (g, c) holds q[head c][32*ks + 8g + e], scaled, hi/lo.
  vec qh[KS], ql[KS];
  {
    const bool live = c < hc;
    const float* qrow = p.q + ((long long)b * p.n_head + hq0 + (live ? c : 0)) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      float x[8];
      const f32x4 a = *(const f32x4*)(qrow + 32 * ks + 8 * g);
      const f32x4 bb = *(const f32x4*)(qrow + 32 * ks + 8 * g + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = live ? a[e] * p.scale_log2 : 0.f;
        x[e + 4] = live ? bb[e] * p.scale_log2 : 0.f;
      }
      split_hi_lo<DT>(x, qh[ks], ql[ks]);
    }
  }

  const long long base = (long long)b * p.batch_stride + (long long)kvh * D * p.max_len;
  const uint16_t* K = (const uint16_t*)p.k + base;
  const uint16_t* V = (const uint16_t*)p.v + base;
  uint16_t* kt = (uint16_t*)lds_raw + wave * D * PITCH;

  f32x4 o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) o[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  for (int t0 = s0 + wave * 32; t0 < s1; t0 += 128) {
    // Issue K tile loads (row = lane/4 + 16*r, 8 columns at 8*(lane&3)) and
    // the V operand loads (row 16*nb + c, columns t0+8g .. +7).
    u16x8 kr[D / 16];
#pragma unroll
    for (int r = 0; r < D / 16; ++r) {
      const int row = (lane >> 2) + 16 * r;
      kr[r] = load_row8<VEC>(K + (long long)row * p.max_len, t0 + 8 * (lane & 3), s1);
    }
    u16x8 vr[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      vr[nb] = load_row8<VEC>(V + (long long)(16 * nb + c) * p.max_len, t0 + 8 * g, s1);

#pragma unroll
    for (int r = 0; r < D / 16; ++r) {
      const int row = (lane >> 2) + 16 * r;
      *(u16x8*)(kt + row * PITCH + 8 * (lane & 3)) = kr[r];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // S^T for the two 16-row halves: row r of half mb is column 8*(r/4) + 4*mb + r%4.
    f32x4 s[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      s[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int tc = 8 * (c >> 2) + 4 * mb + (c & 3);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        u16x8 a;
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = kt[(32 * ks + 8 * g + e) * PITCH + tc];
        const vec av = __builtin_bit_cast(vec, a);
        s[mb] = MfmaT<DT>::mma(av, qh[ks], s[mb]);
        s[mb] = MfmaT<DT>::mma(av, ql[ks], s[mb]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // Lane (g, c) now holds scores of head c for columns t0 + 8g + e,
    // e = 4*mb + i.  Online softmax per head (column c of the MFMA output).
    float sc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = s[e >> 2][e & 3];
      sc[e] = (t0 + 8 * g + e < s1) ? v : -INFINITY;
    }
    float mt = sc[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mt = fmaxf(mt, sc[e]);
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mn = fmaxf(m_run, mt);
    const float alpha = fast_exp2(m_run - mn);
    m_run = mn;
    float pe[8], ps = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pe[e] = fast_exp2(sc[e] - mn);
      ps += pe[e];
    }
    l_run = l_run * alpha + ps;
    vec ph, pl;
    split_hi_lo<DT>(pe, ph, pl);

    // Output rows held by this lane are heads 4g+i: fetch their alphas.
    float ar[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[nb][i] *= ar[i];
      const vec bv = __builtin_bit_cast(vec, vr[nb]);
      o[nb] = MfmaT<DT>::mma(ph, bv, o[nb]);
      o[nb] = MfmaT<DT>::mma(pl, bv, o[nb]);
    }
  }

  // Wave state -> LDS, then the 4-wave merge.
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  __syncthreads();  // K tiles are dead; reuse LDS for the merge buffers
  float* sm_m = (float*)lds_raw;
  float* sm_l = sm_m + 4 * HS;
  float* sm_o = sm_l + 4 * HS;
  if (g == 0) {
    sm_m[wave * HS + c] = m_run;
    sm_l[wave * HS + c] = l_run;
  }
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int i = 0; i < 4; ++i) sm_o[(wave * HS + 4 * g + i) * D + 16 * nb + c] = o[nb][i];
  __syncthreads();
  merge_waves_and_store<D>(p, sm_m, sm_l, sm_o, hc, b, hq0, split, HS);
}

// Folds the partials of all splits: one workgroup per (query head, sequence).
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeParams p) {
  const int hq = blockIdx.x, b = blockIdx.y;
  const int D = p.head_dim, S = p.num_splits;
  const long long row = (long long)b * p.n_head + hq;
  const float* ml = p.ws_ml + row * S * 2;
  __shared__ float sf[1024];
  __shared__ float sinvl;
  float M = -INFINITY;
  for (int s = 0; s < S; ++s) M = fmaxf(M, ml[2 * s]);
  // per-split weights (S <= 1024 enforced on the host)
  for (int s = threadIdx.x; s < S; s += blockDim.x)
    sf[s] = (M == -INFINITY) ? 0.f : fast_exp2(ml[2 * s] - M);
  __syncthreads();
  if (threadIdx.x == 0) {
    float l = 0.f;
    for (int s = 0; s < S; ++s) l += sf[s] * ml[2 * s + 1];
    sinvl = 1.f / l;
  }
  __syncthreads();
  const float* wo = p.ws_o + row * S * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float o = 0.f;
    for (int s = 0; s < S; ++s) o += sf[s] * wo[(long long)s * D + d];
    p.out[row * D + d] = o * sinvl;
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
static int pick_splits(const hl_decode_args* a, int n_chunks, int tile_cols) {
  if (a->num_splits > 0) return a->num_splits;
  const int cols_per_iter = 4 * tile_cols;  // 4 waves
  const long long units = (long long)a->batch * a->n_head_kv * n_chunks;
  const int target = 2048;  // ~8 workgroups per CU on 256 CUs
  int s = (int)((target + units - 1) / units);
  const int max_s = (a->seq_len + cols_per_iter - 1) / cols_per_iter;
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  if (s > 1024) s = 1024;
  return s;
}

void decode_plan(const hl_decode_args* a, DecodePlan* plan) {
  const int G = a->n_head / a->n_head_kv;
  plan->head_chunk = G < 16 ? G : 16;
  plan->n_chunks = (G + plan->head_chunk - 1) / plan->head_chunk;
  const int tile = a->kv_dtype == HL_F32 ? 64 : 32;
  plan->num_splits = pick_splits(a, plan->n_chunks, tile);
  const int per = 4 * tile;
  int split_len = (a->seq_len + plan->num_splits - 1) / plan->num_splits;
  split_len = (split_len + per - 1) / per * per;
  plan->split_len = split_len;
  plan->num_splits = (a->seq_len + split_len - 1) / split_len;
  plan->ws_bytes = plan->num_splits > 1
                       ? (size_t)a->batch * a->n_head * plan->num_splits * (a->head_dim + 2) * 4
                       : 0;
}

hipError_t decode_launch(const hl_decode_args* a, const DecodePlan* plan, void* ws,
                         hipStream_t stream, bool vec_ok) {
  DecodeParams p;
  const int D = a->head_dim;
  p.q = a->q;
  p.k = a->k_cache;
  p.v = a->v_cache;
  p.out = a->out;
  p.ws_o = (float*)ws;
  p.ws_ml = ws ? (float*)ws + (size_t)a->batch * a->n_head * plan->num_splits * D : nullptr;
  p.seq_lens = a->seq_lens;
  p.batch_stride = a->cache_batch_stride ? a->cache_batch_stride
                                         : (long long)a->n_head_kv * D * a->max_len;
  p.n_head = a->n_head;
  p.n_head_kv = a->n_head_kv;
  p.head_dim = D;
  p.group = a->n_head / a->n_head_kv;
  p.head_chunk = plan->head_chunk;
  p.n_chunks = plan->n_chunks;
  p.max_len = a->max_len;
  p.seq_len = a->seq_len;
  p.split_len = plan->split_len;
  p.num_splits = plan->num_splits;
  p.direct = plan->num_splits == 1;
  const float scale = a->scale != 0.f ? a->scale : 1.0f / sqrtf((float)D);
  p.scale_log2 = scale * kLog2e;

  dim3 grid(plan->num_splits, a->n_head_kv * plan->n_chunks, a->batch);
  dim3 block(256);
#define HL_DEC_F32(DD) \
  case DD: hipLaunchKernelGGL(decode_f32_kernel<DD>, grid, block, 0, stream, p); break;
#define HL_DEC_MFMA(DD, DTT)                                                                 \
  case DD:                                                                                   \
    if (vec_ok) hipLaunchKernelGGL((decode_mfma_kernel<DD, DTT, true>), grid, block, 0, stream, p); \
    else hipLaunchKernelGGL((decode_mfma_kernel<DD, DTT, false>), grid, block, 0, stream, p);      \
    break;
  if (a->kv_dtype == HL_F32) {
    switch (D) {
      HL_DEC_F32(64)
      HL_DEC_F32(128)
      default: return hipErrorInvalidValue;
    }
  } else if (a->kv_dtype == HL_F16) {
    switch (D) {
      HL_DEC_MFMA(64, HL_F16)
      HL_DEC_MFMA(128, HL_F16)
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (D) {
      HL_DEC_MFMA(64, HL_BF16)
      HL_DEC_MFMA(128, HL_BF16)
      default: return hipErrorInvalidValue;
    }
  }
#undef HL_DEC_F32
#undef HL_DEC_MFMA
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.direct) return e;
  hipLaunchKernelGGL(decode_merge_kernel, dim3(a->n_head, a->batch), dim3(128), 0, stream, p);
  return hipGetLastError();
}

}  // namespace hl
