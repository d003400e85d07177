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
// (running max m, sum l, accumulators o) in registers and prefetches its next
// tile while computing the current one.  The four waves merge through LDS and
// the workgroup writes one partial (m, l, o[D]) per query head.  The last
// workgroup of a (sequence, kv head, head chunk) to finish folds the partials
// of all splits and writes the output, so one launch does the whole step.
//
// Softmax runs in base 2 (scores pre-multiplied by scale*log2 e), so
// p = exp2(s - m) equals the reference's expf(score - max).
#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "headvec.h"
#include "launch.h"

namespace hl {

// Timing instrumentation for development builds only (-DHL_STAMPS): thread 0
// of every workgroup records s_memrealtime (100 MHz) at entry (0), the first
// tile (1), the end of its streaming loop (2), after the 4-wave merge (3),
// after its arrival (4) and, in the merging workgroup, after the fold (5).
#ifdef HL_STAMPS
__device__ unsigned long long hl_stamps[65536 * 8];
#define HL_STAMP(i)                                                                                  \
  do {                                                                                               \
    const unsigned wg_ = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);            \
    if (threadIdx.x == 0 && wg_ < 65536u) hl_stamps[wg_ * 8 + (i)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define HL_STAMP(i) ((void)0)
#endif

// Workspace layout (num_splits > 1):
//   slots [(b*Hkv + kvh)*n_chunks + chunk]    uint32 arrival counters (first)
//   ws_o  [((b*Hq + hq)*S + split)*D + d]     unnormalised sum p*v
//   ws_ml [((b*Hq + hq)*S + split)*2 + {0,1}] running max (log2 units), sum
// The counters must be zero before the first call (hl_attn_decode_workspace_init);
// the last arrival of every (sequence, kv head, chunk) resets its counter to
// 0, so the workspace is ready for the next call (and for graph replays).
struct DecodeParams {
  const float* q;
  const void* k;
  const void* v;
  float* out;
  float* ws_o;
  float* ws_ml;
  unsigned int* slots;
  const int* seq_lens;
  long long batch_stride;
  int n_head, n_head_kv, head_dim, group, head_chunk, n_chunks;
  int max_len, seq_len, split_len, num_splits;
  int kv_layout;  // HL_KV_COLMAJOR | HL_KV_TILED32 | HL_KV_PAGED32 (the last two: VEC kernels only)
  const int* block_table;  // HL_KV_PAGED32: [B][bps] page of each 32-column tile
  int bps;
  float scale_log2;
  // Fused decode step (STEP kernels only): q above is the raw new-token
  // activation; k_act / v_act are the new token's k and v.  The kernel applies
  // qkNorm + RoPE at column pos = L - 1, writes k / v into that cache column
  // and attends over [0, L), L = (positions ? positions[b] : pos) + 1.
  const float* k_act;
  const float* v_act;
  const float* q_norm_w;
  const float* k_norm_w;
  float eps;
  int rope_dim, rope_style, pos;
  const int* positions;
  ThetaTable theta;
};

constexpr int kMaxFusedSplits = 256;
constexpr long long kPagedMaxSplit = 32768;  // columns per split of a paged cache

// Attention length of sequence b: the new token's column + 1 in a decode
// step with per-sequence positions, else seq_lens[b] or seq_len.
__device__ __forceinline__ int attn_len(const DecodeParams& p, int b) {
  return p.positions ? p.positions[b] + 1 : (p.seq_lens ? p.seq_lens[b] : p.seq_len);
}

// Cross-workgroup exchange of the split partials.  The partials are small, so
// they are written and read with relaxed agent-scope atomic stores/loads
// (write-through / cache-bypassing accesses that are coherent across the
// XCDs' separate L2s) instead of release/acquire fences, which on gfx950
// write back and invalidate the whole L2 of the XCD for every workgroup.
// Ordering: each thread waits for its partial stores to complete
// (s_waitcnt vmcnt(0)) before the workgroup barrier that precedes the
// arrival RMW; the merging workgroup issues its loads only after the RMW has
// returned "last".
__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);  // no compiler reordering across
  __builtin_amdgcn_s_waitcnt(0x0F70);        // s_waitcnt vmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Registers this workgroup's partial; returns true in the last arrival.
__device__ __forceinline__ bool arrive_last(unsigned int* slot, int S) {
  __shared__ int s_last;
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned int old = __hip_atomic_fetch_add(slot, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = old == (unsigned int)(S - 1);
  }
  __syncthreads();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return s_last != 0;
}

// Workgroup epilogue shared by both kernels.  sm_m[w][h], sm_l[w][h] and
// sm_o[w][h][D] hold the 4 waves' states for the hc heads of this chunk.
// `after` runs once the workgroup's partial is registered (or its output
// written): work whose stores must not delay the arrival.
struct NoTail {
  __device__ void operator()() const {}
};
template <int D, typename Tail = NoTail>
__device__ void finish_workgroup(const DecodeParams& p, const float* sm_m, const float* sm_l,
                                 const float* sm_o, int hc, int b, int kvh, int chunk, int hq0,
                                 int split, int hstride, Tail after = Tail()) {
  const int tid = threadIdx.x;
  const int S = p.num_splits;
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
    const long long row = (long long)b * p.n_head + hq0 + h;
    if (S == 1) {
      p.out[row * D + d] = o / l;
    } else {
      const long long pi = row * S + split;
      store_agent(&p.ws_o[pi * D + d], o);
      if (d == 0) {
        store_agent(&p.ws_ml[pi * 2 + 0], M);
        store_agent(&p.ws_ml[pi * 2 + 1], l);
      }
    }
  }
  if (S == 1) {
    after();
    return;
  }
  unsigned int* slot = p.slots + ((long long)b * p.n_head_kv + kvh) * p.n_chunks + chunk;
  const bool last = arrive_last(slot, S);
  HL_STAMP(4);
  after();
  if (!last) return;

  // Fold all splits, 8 at a time: each chunk's m, l and o loads are issued
  // together (one memory round trip per 8 splits), then merged into a
  // running (max, sum, accumulator) per output element.
  for (int idx = tid; idx < hc * D; idx += 256) {
    const int h = idx / D, d = idx % D;
    const long long row = (long long)b * p.n_head + hq0 + h;
    const float* ml = p.ws_ml + row * S * 2;
    const float* wo = p.ws_o + row * S * D + d;
    float M = -INFINITY, lsum = 0.f, osum = 0.f;
    for (int s0 = 0; s0 < S; s0 += 8) {
      float m[8], l[8], x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int sp = min(s0 + u, S - 1);
        m[u] = load_agent(&ml[2 * sp]);
        l[u] = load_agent(&ml[2 * sp + 1]);
        x[u] = load_agent(&wo[(long long)sp * D]);
      }
      float mc = M;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s0 + u < S) mc = fmaxf(mc, m[u]);
      if (mc == -INFINITY) continue;  // no columns so far (empty splits)
      const float r = fast_exp2(M - mc);
      lsum *= r;
      osum *= r;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (s0 + u < S) {
          const float w = fast_exp2(m[u] - mc);
          lsum += w * l[u];
          osum += w * x[u];
        }
      }
      M = mc;
    }
    p.out[row * D + d] = osum / lsum;
  }
  HL_STAMP(5);
  if (tid == 0) __hip_atomic_store(slot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// fp32 KV path (vector ALU).  A wave owns 64 consecutive columns per tile,
// lane j scores column t0+j for every head of the chunk, then lanes switch to
// owning output dims for the P.V product.
// ---------------------------------------------------------------------------
// HC: head slots per chunk (1, 2, 4, 8 or 16, at least the chunk's heads).  Slots
// past the chunk's heads score a zero q row and are never written out; every
// slot is computed without a branch, so the heads' dependency chains (dot
// products, wave reductions) interleave instead of running one after another.
template <int D, bool V4, int HC>
__global__ __launch_bounds__(256) void decode_f32_kernel(DecodeParams p) {
  // D = 128 keeps one head at a time (uniform branches): interleaving every
  // head's chains there needs more registers than the kernel has.
  constexpr bool SEQ = D > 64;
  constexpr int DPL = (D + 63) / 64;  // output dims per lane
  constexpr int MERGE_FLOATS = 4 * HC * (D + 2);
  constexpr int FUSE_FLOATS = 16 * kMaxFusedSplits + 16;
  constexpr int SM_FLOATS = MERGE_FLOATS > FUSE_FLOATS ? MERGE_FLOATS : FUSE_FLOATS;
  __shared__ __attribute__((aligned(16))) float sq[HC * D];
  __shared__ __attribute__((aligned(16))) float sp[4][HC][64];
  __shared__ __attribute__((aligned(16))) float sm[SM_FLOATS];

  HL_STAMP(0);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches
  const int b = blockIdx.z;
  const int kvh = blockIdx.y / p.n_chunks, chunk = blockIdx.y % p.n_chunks;
  const int hq0 = kvh * p.group + chunk * p.head_chunk;
  const int hc = min(p.head_chunk, p.group - chunk * p.head_chunk);
  const int split = blockIdx.x;
  const int L = attn_len(p, b);
  const int s0 = split * p.split_len;
  const int s1 = split == p.num_splits - 1 ? L : min(L, s0 + p.split_len);  // last split takes the rest

  const long long base = (long long)b * p.batch_stride + (long long)kvh * D * p.max_len;
  const float* K = (const float*)p.k + base;
  const float* V = (const float*)p.v + base;

  // A wave owns 64 consecutive columns per tile: lane j scores column t0+j
  // for every head, then lanes switch to owning output dims d = lane + 64i
  // for the P.V product.  Every global load of a tile (the first K column
  // batch, coalesced across lanes, and the lane's V rows) is issued before
  // any is used: one memory round trip per tile, not one per element.  The
  // first tile's loads go out before q is staged, so they overlap it.
  float kv[64], vv[DPL][64];
  auto load_tile = [&](int t0) {
    const int colc = min(t0 + lane, s1 - 1);  // in bounds; scores of lanes past s1 are dropped
#pragma unroll
    for (int u = 0; u < 64; ++u) kv[u] = K[(long long)u * p.max_len + colc];
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      const float* vrow = V + (long long)(lane + 64 * i) * p.max_len;
      if constexpr (V4) {
#pragma unroll
        for (int c4 = 0; c4 < 16; ++c4) {
          const f32x4 x = *(const f32x4*)(vrow + min(t0 + 4 * c4, p.max_len - 4));
#pragma unroll
          for (int e = 0; e < 4; ++e) vv[i][4 * c4 + e] = x[e];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 64; ++j) vv[i][j] = vrow[min(t0 + j, s1 - 1)];
      }
    }
  };
  int t0 = s0 + wave * 64;
  if (t0 < s1) load_tile(t0);

  const float* qb = p.q + ((long long)b * p.n_head + hq0) * D;
  for (int i = tid; i < HC * D; i += 256) {
    const int h = i / D;
    sq[i] = h < hc ? qb[i] : 0.f;
  }
  __syncthreads();

  float m_run[HC], l_run[HC], acc[HC][DPL];
#pragma unroll
  for (int h = 0; h < HC; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[h][i] = 0.f;
  }

  HL_STAMP(1);
  for (bool first = true; t0 < s1; t0 += 256, first = false) {
    if (!first) load_tile(t0);
    const int col = t0 + lane;
    const bool valid = col < s1;
    const int colc = valid ? col : s1 - 1;
    float s[HC];
#pragma unroll
    for (int h = 0; h < HC; ++h) s[h] = 0.f;
#pragma unroll
    for (int db = 0; db < D / 64; ++db) {
      if (db > 0) {
#pragma unroll
        for (int u = 0; u < 64; ++u) kv[u] = K[(long long)(64 * db + u) * p.max_len + colc];
      }
#pragma unroll
      for (int h = 0; h < HC; ++h) {
        if (SEQ && h >= hc) continue;  // uniform
#pragma unroll
        for (int u = 0; u < 64; u += 4) {
          const f32x4 qv = *(const f32x4*)&sq[h * D + 64 * db + u];
#pragma unroll
          for (int e = 0; e < 4; ++e) s[h] = fmaf(qv[e], kv[u + e], s[h]);
        }
      }
    }
    // score = dot * scale (naive.nim:3328), here in log2 units
    float alpha[HC], sv[HC], mt[HC];
#pragma unroll
    for (int h = 0; h < HC; ++h) mt[h] = sv[h] = valid ? s[h] * p.scale_log2 : -INFINITY;
    if constexpr (SEQ) {
#pragma unroll
      for (int h = 0; h < HC; ++h)
        if (h < hc) mt[h] = wave_max(mt[h]);
    } else {  // wave max of every head, the butterflies of all heads interleaved
#pragma unroll
      for (int o = 32; o > 0; o >>= 1)
#pragma unroll
        for (int h = 0; h < HC; ++h) mt[h] = fmaxf(mt[h], __shfl_xor(mt[h], o, 64));
    }
#pragma unroll
    for (int h = 0; h < HC; ++h) {
      if (SEQ && h >= hc) {
        alpha[h] = 1.f;
        continue;
      }
      const float mn = fmaxf(m_run[h], mt[h]);
      alpha[h] = fast_exp2(m_run[h] - mn);
      const float pv = fast_exp2(sv[h] - mn);
      m_run[h] = mn;
      l_run[h] = l_run[h] * alpha[h] + pv;  // per-lane partial, summed at the end
      sp[wave][h][lane] = pv;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int nj = min(64, s1 - t0);
#pragma unroll
    for (int i = 0; i < DPL; ++i)
#pragma unroll
      for (int j = 0; j < 64; ++j) vv[i][j] = j < nj ? vv[i][j] : 0.f;
#pragma unroll
    for (int h = 0; h < HC; ++h) {
      if (SEQ && h >= hc) continue;
#pragma unroll
      for (int i = 0; i < DPL; ++i) acc[h][i] *= alpha[h];
#pragma unroll
      for (int j = 0; j < 64; j += 4) {
        const f32x4 pw = *(const f32x4*)&sp[wave][h][j];
#pragma unroll
        for (int i = 0; i < DPL; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[h][i] = fmaf(pw[e], vv[i][j + e], acc[h][i]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  HL_STAMP(2);
  float* sm_m = sm;
  float* sm_l = sm_m + 4 * HC;
  float* sm_o = sm_l + 4 * HC;
  float lsum[HC];
#pragma unroll
  for (int h = 0; h < HC; ++h) lsum[h] = l_run[h];
  if constexpr (SEQ) {
#pragma unroll
    for (int h = 0; h < HC; ++h)
      if (h < hc) lsum[h] = wave_sum(lsum[h]);
  } else {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
#pragma unroll
      for (int h = 0; h < HC; ++h) lsum[h] += __shfl_xor(lsum[h], o, 64);
  }
#pragma unroll
  for (int h = 0; h < HC; ++h) {
    const float l = lsum[h];
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
  HL_STAMP(3);
  finish_workgroup<D>(p, sm_m, sm_l, sm_o, hc, b, kvh, chunk, hq0, split, HC);
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
// VEC (rows 16-byte aligned, max_len % 8 == 0): one unconditional 16-byte
// load at a column clamped into the row, so every wave issues the same loads
// and the compiler can wait on exact counts; masking happens after the load.
template <bool VEC>
__device__ __forceinline__ u16x8 load_row8(const uint16_t* row, int col, int lim, int max_len) {
  u16x8 r;
  if (VEC) {
    r = *(const u16x8*)(row + min(col, max_len - 8));
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (col + e < lim) ? row[col + e] : (uint16_t)0;
  }
  return r;
}
__device__ __forceinline__ u16x8 mask_row8(u16x8 r, int col, int lim) {
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (col + e < lim) ? r[e] : (uint16_t)0;
  return r;
}

// PG: paged caches (a compile-time variant, so the other layouts carry no
// page lookups).
// Launch bounds: the prefetching kernels hold two tiles per wave (one
// workgroup per CU at head dim 128); the others fill more workgroups per CU
// where their registers allow it without spilling.  Measured against the
// tighter bounds that spilled: the fused step at head dim 128 (Llama-3-8B-
// shaped layer, one sequence, 2K columns) 15.3 -> 13.0 us; the scalar-load
// kernel at head dim 64 (c3 shape with an odd cache length) 40.5 -> 28.8 us.
template <int D, int DT, bool VEC, bool PIPE, bool STEP, bool PG = false>
__global__ __launch_bounds__(256, PIPE ? (D == 64 ? 2 : 1) : (D == 64 ? (VEC ? 4 : 2) : (STEP ? 1 : 2))) void decode_mfma_kernel(DecodeParams p) {
  static_assert(!PG || VEC, "paged caches are read with vector loads only");
  // MFMA operand type: the storage type, except fp8 caches, which are
  // converted to fp16 (exactly) as their tiles arrive.
  constexpr int MT = DT == HL_FP8 ? HL_F16 : DT;
  static_assert(DT != HL_FP8 || VEC, "fp8 caches are read with vector loads only");
  typedef typename MfmaT<MT>::vec vec;
  typedef typename std::conditional<DT == HL_FP8, uint8_t, uint16_t>::type elem_t;
  // Tile registers hold what the loads return: 8 fp16/bf16 values per row
  // chunk, or for fp8 the 8 raw bytes, converted when the tile is computed
  // (converting at load time would wait for the loads there).
  typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
  typedef typename std::conditional<DT == HL_FP8, u32x2v, u16x8>::type raw_t;
  constexpr int KS = D / 32;      // k-steps of the QK^T product
  constexpr int NB = D / 16;      // 16-dim output blocks
  constexpr int KR = D / 16;      // 16-byte K loads per lane per tile
  // LDS row pitch (elements) of a 32-column K tile: 72 bytes, so that the
  // gathers of one MFMA operand (rows 8 apart) fall in distinct banks; rows
  // are 8-byte aligned and written as two 8-byte halves per 16-byte chunk.
  constexpr int PITCH = 36;
  constexpr int HS = 16;          // head slots of the merge buffers
  constexpr int KT_BYTES = 4 * D * PITCH * 2;                   // 4 wave tiles (uint16)
  constexpr int MERGE_BYTES = 4 * HS * (D + 2) * 4;
  constexpr int FUSE_BYTES = (16 * kMaxFusedSplits + 16) * 4;
  constexpr int LDS_A = KT_BYTES > MERGE_BYTES ? KT_BYTES : MERGE_BYTES;
  constexpr int LDS_BYTES = LDS_A > FUSE_BYTES ? LDS_A : FUSE_BYTES;
  static_assert(18 * D * 4 <= LDS_BYTES, "step prologue buffers alias the K tiles");
  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[LDS_BYTES];
  __shared__ uint16_t snew[STEP ? 2 * D : 1];  // new column's k, v in storage bits

  HL_STAMP(0);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches
  const int g = lane >> 4, c = lane & 15;
  const int b = blockIdx.z;
  const int kvh = blockIdx.y / p.n_chunks, chunk = blockIdx.y % p.n_chunks;
  const int hq0 = kvh * p.group + chunk * p.head_chunk;
  const int hc = min(p.head_chunk, p.group - chunk * p.head_chunk);
  const int split = blockIdx.x;
  const int L = attn_len(p, b);
  const int s0 = split * p.split_len;
  const int s_end = split == p.num_splits - 1 ? L : min(L, s0 + p.split_len);  // last split takes the rest
  // Fused step: the new column L - 1 belongs to exactly one split (has_new).
  // Its k / v are computed in this kernel, so that split seeds its softmax
  // state with the column directly and its tiles stop before it.
  const int newc = L - 1;
  const bool has_new = STEP && s0 <= newc && newc < s_end;
  const int s1 = has_new ? newc : s_end;  // end of the columns read from the cache

  // Paged caches: this head's [D][32] block inside every page; the page of
  // each tile comes from the block table (see page_of below).
  constexpr bool paged = PG;
  const long long base = paged ? (long long)kvh * D * 32
                               : (long long)b * p.batch_stride + (long long)kvh * D * p.max_len;
  const elem_t* K = (const elem_t*)p.k + base;
  const elem_t* V = (const elem_t*)p.v + base;
  uint16_t* kt = (uint16_t*)lds_raw + wave * D * PITCH;

  // K tile: row = lane/4 + 16*r, 8 columns at 8*(lane&3); V operand: row
  // 16*nb + c, columns t0+8g .. +7.
  // The scheduling barriers keep each tile's loads together and in program
  // order, so a compute waits only for its own tile, never for loads issued
  // after it.
  // Tiled caches (VEC only): tile t0 / 32 of the head is [D][32] at
  // (t0 / 32) * D * 32, rows 32 elements apart; the address form is selected
  // without a branch so that both layouts issue the same loads.
  // Paged: lane i of register q holds the page of this wave's tile
  // 64q + i (columns s0 + 32*wave + 128*(64q + i)), read with readlane; up
  // to 256 tiles per wave (the plan keeps splits within 32768 columns).
  // Pages past the sequence's last column are never touched (clamped).
  const bool tiled = VEC && (p.kv_layout == HL_KV_TILED32 || paged);
  const int rstride = tiled ? 32 : p.max_len;
  int pg[4] = {0, 0, 0, 0}, pg_first = 0;
  if constexpr (paged) {
    const int* row = p.block_table + (long long)b * p.bps;
    const int first = s0 >> 5, lastp = min((L - 1) >> 5, p.max_len / 32 - 1);
#pragma unroll
    for (int q = 0; q < 4; ++q) pg[q] = row[min(first + wave + 4 * (lane + 64 * q), lastp)];
    pg_first = row[min(first, lastp)];
  }
  const long long page_elems = (long long)p.n_head_kv * D * 32;
  // Element offset of tile t0's [D][32] block (t0 is this wave's own tile,
  // or s0 for a wave that has none: wave-uniform either way).
  auto page_of = [&](int t0) -> long long {
    const int rel = (t0 >> 5) - (s0 >> 5);
    if ((rel & 3) != wave) return (long long)pg_first * page_elems;
    const int i = rel >> 2, q = i >> 6;
    const int v = q == 0 ? pg[0] : (q == 1 ? pg[1] : (q == 2 ? pg[2] : pg[3]));
    return (long long)__builtin_amdgcn_readlane(v, i & 63) * page_elems;
  };
  auto load_tile = [&](int t0, raw_t* kr, raw_t* vr) {
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (VEC) {
      long long tb;
      if constexpr (paged) tb = page_of(t0);
      else tb = tiled ? (long long)(t0 >> 5) * (D * 32) : 0;
      const int ck = tiled ? 8 * (lane & 3) : min(t0 + 8 * (lane & 3), p.max_len - 8);
      const int cv = tiled ? 8 * g : min(t0 + 8 * g, p.max_len - 8);
      if constexpr (DT == HL_FP8) {  // 8-byte loads of 8 e4m3 values
#pragma unroll
        for (int r = 0; r < KR; ++r) {
          const int row = (lane >> 2) + 16 * r;
          kr[r] = *(const u32x2v*)(K + tb + (long long)row * rstride + ck);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) vr[nb] = *(const u32x2v*)(V + tb + (long long)(16 * nb + c) * rstride + cv);
      } else {
#pragma unroll
        for (int r = 0; r < KR; ++r) {
          const int row = (lane >> 2) + 16 * r;
          kr[r] = *(const u16x8*)(K + tb + (long long)row * rstride + ck);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) vr[nb] = *(const u16x8*)(V + tb + (long long)(16 * nb + c) * rstride + cv);
      }
    } else if constexpr (DT != HL_FP8) {
#pragma unroll
      for (int r = 0; r < KR; ++r) {
        const int row = (lane >> 2) + 16 * r;
        kr[r] = load_row8<false>(K + (long long)row * p.max_len, t0 + 8 * (lane & 3), s1, p.max_len);
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        vr[nb] = load_row8<false>(V + (long long)(16 * nb + c) * p.max_len, t0 + 8 * g, s1, p.max_len);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Fused step: the new token's head vectors this workgroup needs are
  // vector j < hc: q head hq0 + j; j == hc: k; j == hc + 1: v (the last two
  // only in the split that holds the new column).  Wave w takes j = w, w+4, ...
  // Every global read of the prologue (the vectors, norm weights, the lane's
  // RoPE frequency) is issued unconditionally before the first tile's loads,
  // so waiting for them never waits for the tile.
  constexpr int DPL = D / 64;  // elements d = lane + 64e of a head vector per lane
  constexpr int VPW = 5;       // vectors per wave: (16 heads + k + v) / 4, rounded up
  const int nvec = hc + (has_new ? 2 : 0);
  float act[STEP ? VPW : 1][DPL], wq[DPL], wk[DPL];
  float theta_lane = 0.f;
  if constexpr (STEP) {
    const float* qb = p.q + ((long long)b * p.n_head + hq0) * D;
    const float* kb_ = p.k_act + ((long long)b * p.n_head_kv + kvh) * D;
    const float* vb_ = p.v_act + ((long long)b * p.n_head_kv + kvh) * D;
#pragma unroll
    for (int u = 0; u < VPW; ++u) {
      const int j = min(wave + 4 * u, nvec - 1);
      const float* src = j < hc ? qb + j * D : (j == hc ? kb_ : vb_);
#pragma unroll
      for (int e = 0; e < DPL; ++e) act[u][e] = src[lane + 64 * e];
    }
    const float* nq = p.q_norm_w ? p.q_norm_w : qb;  // stand-ins keep the loads unconditional
    const float* nk = p.k_norm_w ? p.k_norm_w : qb;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      wq[e] = nq[lane + 64 * e];
      wk[e] = nk[lane + 64 * e];
    }
    theta_lane = p.theta.t[lane];
  }

  // Plain kernel: this lane's q values, also loaded ahead of the tiles.
  const bool live = c < hc;
  f32x4 qraw[STEP ? 1 : 2 * KS];
  if constexpr (!STEP) {
    const float* qrow = p.q + ((long long)b * p.n_head + hq0 + (live ? c : 0)) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qraw[2 * ks] = *(const f32x4*)(qrow + 32 * ks + 8 * g);
      qraw[2 * ks + 1] = *(const f32x4*)(qrow + 32 * ks + 8 * g + 4);
    }
  }

  // Issue the first tile (and, prefetching, the second) unconditionally: a
  // wave with fewer tiles re-reads one it already asked for (a cache hit), so
  // every wait below can count loads exactly.  The second tile's loads go
  // out only once q is ready in the fused step and at head dim 128: every
  // workgroup requests its first tiles at once, and fewer requests in that
  // burst let the prologue's own loads (and, in the step, its barriers)
  // clear sooner (c3 step 12.70 -> 12.05 us, c5 attention 191.1 -> 188.5
  // us; at head dim 64 attention alone is 0.1 us faster with both early).
  int t0 = s0 + wave * 32;
  raw_t ka[KR], va[NB], kb[KR], vb[NB];
  const int ta = t0 < s1 ? t0 : s0;
  const int tnext = t0 + 128 < s1 ? t0 + 128 : ta;
  load_tile(ta, ka, va);
  if constexpr (PIPE && !STEP && D == 64) load_tile(tnext, kb, vb);

  // Fused step prologue: qkNorm + RoPE of this chunk's q heads into LDS, and
  // in the split that holds the new column, of k (and v as is).  That split
  // substitutes the new column into its tile registers (it need not see the
  // cache write), and its chunk-0 workgroup writes the column to the cache.
  // Same arithmetic as the stand-alone per-head kernel (shared helpers).
  float* sq = (float*)lds_raw;  // [16][D] roped q, then [2][D] new k, v
  if constexpr (STEP) {
    float* skv = sq + 16 * D;
    const int half = p.rope_dim / 2;  // <= D/2 <= 64: one pair per lane
    // Evaluated on every lane (lanes >= half discard it), so that the
    // frequency load stays ahead of the tile loads.
    const float angle = (float)newc * theta_lane;
    float cs, sn;
    rope_cs(angle, cs, sn);
#pragma unroll
    for (int u = 0; u < VPW; ++u) {
      const int j = wave + 4 * u;
      if (j < nvec) {
        const bool isq = j < hc, isk = j == hc;
        float x[DPL];
#pragma unroll
        for (int e = 0; e < DPL; ++e) x[e] = act[u][e];
        if ((isq && p.q_norm_w) || (isk && p.k_norm_w)) {
          float ss = 0.f;
#pragma unroll
          for (int e = 0; e < DPL; ++e) ss = sq_acc(ss, x[e]);
          const float inv = rms_inv(ss, D, p.eps);
#pragma unroll
          for (int e = 0; e < DPL; ++e) x[e] = norm_apply(x[e], inv, isq ? wq[e] : wk[e]);
        }
        float* dst = isq ? sq + j * D : skv + (j - hc) * D;
#pragma unroll
        for (int e = 0; e < DPL; ++e) dst[lane + 64 * e] = x[e];
        if (isq || isk) {
          wave_lds_sync();
          if (lane < half) rope_rotate(dst, lane, half, p.rope_style, cs, sn);
        }
      }
    }
    __syncthreads();
    if (has_new) {  // workgroup-uniform
      for (int i = tid; i < 2 * D; i += 256) snew[i] = to_bits<DT>(skv[i]);
      __syncthreads();  // wave 0 seeds from entries the other waves wrote
    }
  }

  // Q^T operand: lane (g, c) holds q[head c][32*ks + 8g + e], scaled, hi/lo.
  vec qh[KS], ql[KS];
  {
    const float* qrow = sq + (live ? c : 0) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      float x[8];
      const f32x4 a = STEP ? *(const f32x4*)(qrow + 32 * ks + 8 * g) : qraw[STEP ? 0 : 2 * ks];
      const f32x4 bb = STEP ? *(const f32x4*)(qrow + 32 * ks + 8 * g + 4) : qraw[STEP ? 0 : 2 * ks + 1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = live ? a[e] * p.scale_log2 : 0.f;
        x[e + 4] = live ? bb[e] * p.scale_log2 : 0.f;
      }
      split_hi_lo<MT>(x, qh[ks], ql[ks]);
    }
  }
  if constexpr (PIPE && !STEP && D != 64) load_tile(tnext, kb, vb);
  f32x4 o[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) o[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  if constexpr (STEP) {
    // Wave 0 of the split holding the new column starts from that column:
    // m = its score, l = 1 (counted once, in lane group 0), o = its v for
    // every head.  The score uses the stored (rounded) k, as a read of the
    // cache would.
    if (has_new && wave == 0) {
      const float* qrow = sq + (live ? c : 0) * D;
      constexpr int DG = D / 4;  // dims per lane group
      float dot = 0.f;
#pragma unroll
      for (int d = 0; d < DG; ++d) dot += qrow[DG * g + d] * from_bits<DT>(snew[DG * g + d]);
      dot += __shfl_xor(dot, 16, 64);
      dot += __shfl_xor(dot, 32, 64);
      m_run = live ? dot * p.scale_log2 : 0.f;
      l_run = g == 0 ? 1.f : 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const float vn = from_bits<DT>(snew[D + 16 * nb + c]);
        o[nb] = f32x4{vn, vn, vn, vn};
      }
    }
    __syncthreads();  // sq is dead; the K tiles reuse its LDS
  }
  if constexpr (PIPE && STEP) load_tile(tnext, kb, vb);
  HL_STAMP(1);

  // One 32-column tile whose K/V registers have been loaded.
  auto compute_tile = [&](int t0, u16x8* kr, u16x8* vr) {
    if (VEC && t0 + 32 > s1) {  // boundary tile (wave-uniform): zero columns >= s1
#pragma unroll
      for (int r = 0; r < KR; ++r) kr[r] = mask_row8(kr[r], t0 + 8 * (lane & 3), s1);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) vr[nb] = mask_row8(vr[nb], t0 + 8 * g, s1);
    }
#pragma unroll
    for (int r = 0; r < KR; ++r) {
      const int row = (lane >> 2) + 16 * r;
      typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
      uint16_t* dst = kt + row * PITCH + 8 * (lane & 3);
      *(u16x4*)dst = u16x4{kr[r][0], kr[r][1], kr[r][2], kr[r][3]};
      *(u16x4*)(dst + 4) = u16x4{kr[r][4], kr[r][5], kr[r][6], kr[r][7]};
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
        s[mb] = MfmaT<MT>::mma(av, qh[ks], s[mb]);
        s[mb] = MfmaT<MT>::mma(av, ql[ks], s[mb]);
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
    split_hi_lo<MT>(pe, ph, pl);

    // Output rows held by this lane are heads 4g+i: fetch their alphas.
    float ar[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[nb][i] *= ar[i];
      const vec bv = __builtin_bit_cast(vec, vr[nb]);
      o[nb] = MfmaT<MT>::mma(ph, bv, o[nb]);
      o[nb] = MfmaT<MT>::mma(pl, bv, o[nb]);
    }
  };

  auto compute = [&](int t0, raw_t* kw, raw_t* vw) {
    if constexpr (DT == HL_FP8) {
      u16x8 kr[KR], vr[NB];
#pragma unroll
      for (int r = 0; r < KR; ++r) kr[r] = e4m3x8_to_f16x8(kw[r][0], kw[r][1]);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) vr[nb] = e4m3x8_to_f16x8(vw[nb][0], vw[nb][1]);
      compute_tile(t0, kr, vr);
    } else {
      compute_tile(t0, kw, vw);
    }
  };

  // PIPE: two buffers, a and b, hold this wave's tiles t0 and t0 + 128
  // (t0, t0+128, ... step 128).  While one computes, the next tile's loads
  // into the other are in flight.  The loop covers the pairs that are
  // followed by a whole pair, so its loads are unconditional and every path
  // into a compute has the same loads outstanding (the compiler's waits then
  // count exactly: a compute waits for its own tile only); the last 2 or 3
  // tiles are finished after it without further speculative loads.
  // !PIPE (about one tile per wave): no second buffer, fewer registers,
  // more resident waves.
  if (!PIPE) {
    if (t0 < s1) {
      compute(t0, ka, va);
      for (t0 += 128; t0 < s1; t0 += 128) {
        load_tile(t0, ka, va);
        compute(t0, ka, va);
      }
    }
  } else {
    const int n_tiles = t0 < s1 ? (s1 - t0 + 127) / 128 : 0;  // wave-uniform
    if (n_tiles >= 2) {
      int i = 0;
      for (; i + 4 <= n_tiles; i += 2, t0 += 256) {
        compute(t0, ka, va);
        load_tile(t0 + 256, ka, va);
        compute(t0 + 128, kb, vb);
        load_tile(t0 + 384, kb, vb);
      }
      if (n_tiles - i == 3) {
        compute(t0, ka, va);
        load_tile(t0 + 256, ka, va);
        compute(t0 + 128, kb, vb);
        compute(t0 + 256, ka, va);
      } else {
        compute(t0, ka, va);
        compute(t0 + 128, kb, vb);
      }
    } else if (n_tiles == 1) {
      compute(t0, ka, va);
    }
  }

  HL_STAMP(2);
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
  HL_STAMP(3);
  if constexpr (STEP) {
    // The new column goes to the cache after this workgroup's arrival, so its
    // stores neither count against the tile waits nor delay the merge, as
    // nontemporal stores: they are scattered 2-byte writes (one per cache
    // row), and written through they leave no dirty partial lines for the
    // end of the kernel to write back (c3 step: 12.78 -> 12.64 us; issued
    // before the tiles instead, the plain stores cost as much, because the
    // tile waits count them).
    finish_workgroup<D>(p, sm_m, sm_l, sm_o, hc, b, kvh, chunk, hq0, split, HS, [&]() {
      if (has_new && chunk == 0) {
        for (int i = tid; i < 2 * D; i += 256) {
          const int dd = i < D ? i : i - D;
          long long at;
          if constexpr (paged) at = kv_paged_off(p.block_table, p.bps, b, p.n_head_kv, kvh, D, dd, newc);
          else at = base + kv_off(p.kv_layout, dd, newc, D, p.max_len);
          if constexpr (DT == HL_FP8)  // snew holds the fp16 form of an e4m3 value: exact
            __builtin_nontemporal_store(f32_to_e4m3(from_bits<DT>(snew[i])), &((uint8_t*)(i < D ? p.k : p.v))[at]);
          else
            __builtin_nontemporal_store(snew[i], &((uint16_t*)(i < D ? p.k : p.v))[at]);
        }
      }
    });
  } else {
    finish_workgroup<D>(p, sm_m, sm_l, sm_o, hc, b, kvh, chunk, hq0, split, HS);
  }
}

// Zero-fills a workspace (a kernel rather than a memset node, so that it can
// be captured in a HIP graph).
__global__ __launch_bounds__(256) void zero_fill_kernel(unsigned int* p, size_t n_words, unsigned char* tail,
                                                        int n_tail) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n_words; i += (size_t)gridDim.x * 256) p[i] = 0u;
  if (blockIdx.x == 0 && (int)threadIdx.x < n_tail) tail[threadIdx.x] = 0;
}

hipError_t zero_fill_launch(void* ws, size_t bytes, hipStream_t stream) {
  const size_t words = bytes / 4;
  const int n_tail = (int)(bytes % 4);
  unsigned int blocks = (unsigned int)((words + 255) / 256);
  if (blocks == 0) blocks = 1;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(zero_fill_kernel, dim3(blocks), dim3(256), 0, stream, (unsigned int*)ws, words,
                     (unsigned char*)ws + words * 4, n_tail);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
// CUs of the current device (cached per device).
int cu_count() {
  static std::mutex mu;
  static std::map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();
    return 256;
  }
  cache[dev] = cus;
  return cus;
}

namespace {

typedef void (*KernelFn)(DecodeParams);

// The prefetching kernel exists for the 16-byte path only (the element-wise
// loads of unaligned caches would not fit its registers).
template <int D, bool V4>
KernelFn pick_f32_hc(int hc) {
  if (hc <= 1) return decode_f32_kernel<D, V4, 1>;
  if (hc <= 2) return decode_f32_kernel<D, V4, 2>;
  return hc <= 4 ? decode_f32_kernel<D, V4, 4> : (hc <= 8 ? decode_f32_kernel<D, V4, 8> : decode_f32_kernel<D, V4, 16>);
}
KernelFn pick_f32(int D, bool vec, int hc) {
  if (vec) return D == 64 ? pick_f32_hc<64, true>(hc) : pick_f32_hc<128, true>(hc);
  return D == 64 ? pick_f32_hc<64, false>(hc) : pick_f32_hc<128, false>(hc);
}

template <int D, int DT, bool STEP>
KernelFn pick_mfma(bool vec, bool pipe, bool paged) {
  if (paged)
    return pipe ? decode_mfma_kernel<D, DT, true, true, STEP, true> : decode_mfma_kernel<D, DT, true, false, STEP, true>;
  if (vec || DT == HL_FP8)  // fp8 caches are tiled or paged: always vector loads
    return pipe ? decode_mfma_kernel<D, DT, true, true, STEP> : decode_mfma_kernel<D, DT, true, false, STEP>;
  if constexpr (DT != HL_FP8) return decode_mfma_kernel<D, DT, false, false, STEP>;
  return nullptr;
}

template <int D, int DT>
KernelFn pick_mfma(bool vec, bool pipe, bool step, bool paged) {
  return step ? pick_mfma<D, DT, true>(vec, pipe, paged) : pick_mfma<D, DT, false>(vec, pipe, paged);
}

KernelFn pick_kernel(int kv_dtype, int D, bool vec, bool pipe, bool step, int hc, bool paged) {
  if (kv_dtype == HL_F32) return pick_f32(D, vec, hc);
  if (kv_dtype == HL_F16)
    return D == 64 ? pick_mfma<64, HL_F16>(vec, pipe, step, paged) : pick_mfma<128, HL_F16>(vec, pipe, step, paged);
  if (kv_dtype == HL_FP8)
    return D == 64 ? pick_mfma<64, HL_FP8>(vec, pipe, step, paged) : pick_mfma<128, HL_FP8>(vec, pipe, step, paged);
  return D == 64 ? pick_mfma<64, HL_BF16>(vec, pipe, step, paged) : pick_mfma<128, HL_BF16>(vec, pipe, step, paged);
}

// Resident workgroups of a kernel on the whole device (cached).
int capacity(KernelFn fn) {
  static std::mutex mu;
  static std::map<std::pair<int, KernelFn>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 512;
  std::lock_guard<std::mutex> lk(mu);
  auto key = std::make_pair(dev, fn);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)fn, 256, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      per_cu <= 0 || cus <= 0) {
    (void)hipGetLastError();
    return 512;
  }
  cache[key] = per_cu * cus;
  return per_cu * cus;
}

bool vec_path(const hl_decode_args* a) {
  const long long stride = a->cache_batch_stride ? a->cache_batch_stride
                                                 : (long long)a->n_head_kv * a->head_dim * a->max_len;
  // 16-byte loads of cache rows: 8 elements (fp16/bf16) or 4 (fp32)
  const int per16 = a->kv_dtype == HL_F32 ? 4 : 8;
  return (a->max_len % per16 == 0) && (stride % per16 == 0) &&
         ((uintptr_t)a->k_cache & 15) == 0 && ((uintptr_t)a->v_cache & 15) == 0;
}

}  // namespace

void decode_plan(const hl_decode_args* a, DecodePlan* plan, bool step) {
  const int G = a->n_head / a->n_head_kv;
  plan->head_chunk = G < 16 ? G : 16;
  if (a->kv_dtype == HL_F32) {
    // fp32 (vector ALU): a wave's work per tile grows with its heads.  When
    // the grid is small (latency-bound: fewer workgroups than CUs), fewer
    // heads per workgroup, down to one, spread the work over more CUs; each
    // chunk re-reads the K/V tile, which such small caches serve from L2
    // (c1: 8 -> 1 head, 12.4 -> 7.5 us; head dim 128, 8 kv heads, 1024
    // columns: 17.2 -> 14.0 us).
    const int tiles64 = (a->seq_len + 63) / 64;
    while (plan->head_chunk > 1) {
      const long long wgs = (long long)a->batch * a->n_head_kv * ((G + plan->head_chunk - 1) / plan->head_chunk) *
                            (tiles64 < 64 ? tiles64 : 64);
      if (wgs >= cu_count()) break;
      plan->head_chunk /= 2;
    }
  }
  plan->n_chunks = (G + plan->head_chunk - 1) / plan->head_chunk;
  plan->vec = vec_path(a);
  plan->step = step && a->kv_dtype != HL_F32;
  const bool mfma = a->kv_dtype != HL_F32;
  const int tile = mfma ? 32 : 64;
  const int tiles = (a->seq_len + tile - 1) / tile;
  const long long units = (long long)a->batch * a->n_head_kv * plan->n_chunks;
  // The prefetching kernel streams best with one workgroup per CU (its own
  // loads in flight hide the latency; more splits only add partials to
  // merge), and is used when that gives each wave at least two tiles (8 per
  // split).  Otherwise the register-light kernel fills one round of resident
  // workgroups.
  auto clamp_splits = [&](long long S) { return (int)(S < 1 ? 1 : (S > tiles ? tiles : S)); };
  const int s_pipe = clamp_splits(cu_count() / units);
  int S;
  if (a->num_splits > 0) {
    S = a->num_splits < tiles ? a->num_splits : tiles;
    plan->pipe = mfma && plan->vec && tiles / S >= 8;
  } else if (mfma && plan->vec && tiles / s_pipe >= 8) {
    plan->pipe = true;
    S = s_pipe;
  } else {
    // One round of resident workgroups; for the MFMA kernel at least one
    // tile per wave in each split: a split of fewer tiles leaves waves idle
    // and only adds a partial to the fold (Llama-3-8B shape, one sequence,
    // 2K columns: 64 one-tile splits, 27.8 us, against 16 splits, 15.2 us).
    plan->pipe = false;
    const long long fill = capacity(pick_kernel(a->kv_dtype, a->head_dim, plan->vec, false, plan->step,
                                                plan->head_chunk, a->kv_layout == HL_KV_PAGED32)) / units;
    S = clamp_splits(mfma ? std::min<long long>(fill, std::max(1, tiles / 4)) : fill);
  }
  if (S > kMaxFusedSplits) S = kMaxFusedSplits;
  // Paged caches: a wave keeps the pages of at most 256 tiles, so no split
  // (the last one takes the remainder) may exceed 32768 columns.
  if (a->kv_layout == HL_KV_PAGED32)
    while (S < tiles && S < kMaxFusedSplits &&
           (long long)a->seq_len - (long long)(S - 1) * (tiles / S) * tile > kPagedMaxSplit)
      ++S;
  const int tiles_per_split = tiles / S;  // the last split also takes the remainder
  plan->split_len = tiles_per_split * tile;
  plan->num_splits = S;
  if (plan->num_splits > 1) {
    // Counters first, in a region sized for the most head chunks any plan
    // of this shape can use (chunks of one head), so that their place depends
    // only on (batch, kv heads, group) and not on the split count or the
    // attention length: a workspace shared by the calls of one model keeps
    // them where the previous call left them (zero).
    const long long max_chunks = G;
    plan->counters_bytes = ((size_t)a->batch * a->n_head_kv * max_chunks * 4 + 255) / 256 * 256;
    const size_t partial = (size_t)a->batch * a->n_head * plan->num_splits * (a->head_dim + 2) * 4;
    plan->ws_bytes = plan->counters_bytes + partial;
  } else {
    plan->counters_bytes = 0;
    plan->ws_bytes = 0;
  }
}

hipError_t decode_launch(const hl_decode_args* a, const DecodePlan* plan, void* ws,
                         hipStream_t stream, const DecodeStep* step) {
  DecodeParams p;
  memset(&p, 0, sizeof(p));
  if (step) {
    p.k_act = step->k;
    p.v_act = step->v;
    p.q_norm_w = step->q_norm_w;
    p.k_norm_w = step->k_norm_w;
    p.eps = step->eps;
    p.rope_dim = step->rope_dim;
    p.rope_style = step->rope_style;
    p.pos = step->pos;
    p.positions = step->positions;
    p.theta = step->theta;
  }
  const int D = a->head_dim;
  p.q = a->q;
  p.k = a->k_cache;
  p.v = a->v_cache;
  p.out = a->out;
  p.slots = (unsigned int*)ws;
  p.ws_o = ws ? (float*)((char*)ws + plan->counters_bytes) : nullptr;
  p.ws_ml = ws ? p.ws_o + (size_t)a->batch * a->n_head * plan->num_splits * D : nullptr;
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
  p.kv_layout = a->kv_layout;
  p.block_table = a->block_table;
  p.bps = a->blocks_per_seq;
  p.seq_len = a->seq_len;
  p.split_len = plan->split_len;
  p.num_splits = plan->num_splits;
  const float scale = a->scale != 0.f ? a->scale : 1.0f / sqrtf((float)D);
  p.scale_log2 = scale * kLog2e;

  dim3 grid(plan->num_splits, a->n_head_kv * plan->n_chunks, a->batch);
  KernelFn fn = pick_kernel(a->kv_dtype, D, plan->vec, plan->pipe, plan->step, plan->head_chunk,
                            a->kv_layout == HL_KV_PAGED32);
  hipLaunchKernelGGL(fn, grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace hl

#ifdef HL_STAMPS
extern "C" int hl_debug_stamps(void* host, size_t bytes) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(hl::hl_stamps), bytes);
}
#endif
