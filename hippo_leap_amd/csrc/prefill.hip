// Causal prefill attention for gfx950 (flash-style, online softmax).
//
// Semantics: attentionPrefillKernel / gpuAttentionPrefill (backends/naive.nim:
// 3385-3464): for query row i of head h, scores s_j = (q_i . k_j) * scale for
// j <= i, p = softmax(s), o_i = sum_j p_j v_j; kv head = h / (Hq/Hkv).  The
// reference materialises the whole causal row in a 4096-float LDS array (so
// T <= 4096) and re-reads K/V for every query row; here K/V tiles are staged
// once per workgroup and reused by every query row and every head of the GQA
// group it holds, with no length cap.
//
// Two kernels:
//  * prefill_mfma_kernel: fp16 MFMA (v_mfma_f32_32x32x16_f16) for bf16/fp16
//    activations, on K/V operands prepared by the prologue (kt[Hkv][Tp][D],
//    vt[Hkv][D][Tp]) and Q built in the kernel (or qt[Hq][Tp][D]).  fp16
//    operands keep 11 significant bits (bf16 has 8), which keeps the result
//    within 2e-3 of the fp32 reference; P is rounded to fp16, accumulation
//    is fp32.
//  * prefill_f32mfma_kernel: fp32 MFMA (v_mfma_f32_32x32x2_f32) on the
//    reference's col-major fp32 tensors (the 1e-4 path) in the fallback
//    pass of an MFMA prefill; otherwise fp16 MFMAs on hi/lo splits of the
//    operands, with K and V split once per call by the prologue
//    (prologue_kernel).
#include "common.h"
#include "launch.h"

namespace hl {

// ===========================================================================
// MFMA path
// ===========================================================================
namespace {
constexpr int BN = 64;          // key columns per tile
constexpr int QR = 32;          // query rows per wave
// Lazy rescale: exponents are taken against a reference max that is only
// raised when a row's max exceeds it by more than kRescale (log2 units), so
// P <= 2^kRescale stays well inside fp16 and the O rescale is rare.
constexpr float kRescale = 8.0f;
}  // namespace


int prefill_mfma_tpad(int seq_len) { return (seq_len + BN - 1) / BN * BN; }

struct MfmaPrefillParams {
  const uint16_t* qt;
  const uint16_t* kt;
  const uint16_t* vt;
  void* out;
  int n_head, n_head_kv, group, T, Tp;
  int nh;          // heads per workgroup (8 waves split nh x (8/nh) row blocks)
  int rows_wg;     // query rows per workgroup = 32 * (4/nh)
  int n_qblk;      // query row blocks of rows_wg
  int n_hgrp;      // head groups of nh per kv head
  // Q built in the kernel (QIN != 0): raw col-major q [Hq*D, T]
  const uint16_t* q_in;
  const float* q_norm_w;
  float eps, qscale;  // qscale = scale * log2 e
  int do_rope, rope_dim, rope_style;
  const float2* rope_tab;  // [rope_dim/2][T] (cos, sin)
  unsigned* range_flag;    // see PrefillLaunch
};

__device__ __forceinline__ f32x16 mma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void global_cvoid_t;

// One 16-byte global -> LDS copy per lane; the LDS destination is
// dst + 16 * lane (dst uniform across the wave).  No VGPRs are involved and
// completion is tracked by vmcnt.
__device__ __forceinline__ void copy16_to_lds(const void* src, void* dst_uniform) {
  __builtin_amdgcn_global_load_lds((global_cvoid_t*)src, (lds_void_t*)dst_uniform, 16, 0, 0);
}

// MFMA output row m of a 32-row S^T block holds key sigma(m), where sigma
// permutes groups of 4 rows: with m = 8a + 4h + e,
// sigma(m) = 16*(a>>1) + 8h + 4*(a&1) + e.  The 32x32 MFMA output gives lane
// half h the rows {8a + 4h + e}; under sigma those become, for each 16-key
// k-step u (a = 2u, 2u+1), the 8 consecutive keys 16u + 8h .. 16u + 8h + 7,
// which is exactly one 16-byte chunk of a V row: the P^T operand and the V
// operand need no further shuffling.
__device__ __forceinline__ int sigma_row(int m) {
  const int a = m >> 3, h = (m >> 2) & 1, e = m & 3;
  return 16 * (a >> 1) + 8 * h + 4 * (a & 1) + e;
}

// Q^T operand of one wave built from the raw activations: lane (ln, hh) holds
// q[t = r0 + ln][16k + 8hh + e] after optional qkNorm (RMSNorm over the head
// dimension: the lane's 64 values plus the other half via one xor-32
// exchange) and RoPE, times scale * log2 e, rounded to fp16.  RoPE partners
// are in the same lane: half-split over the full head dimension pairs dims
// d and d + D/2 (k-steps k and k + KSTEPS/2), interleaved pairs e and e + 1.
// Same formulas as the stand-alone prologue: x * (1/sqrtf(ss/D + eps)) * w[d],
// (v0, v1) -> (v0*c - v1*s, v0*s + v1*c).
template <int D, int QDT>
__device__ __forceinline__ void build_q(const MfmaPrefillParams& p, int hq, int r0, int ln, int hh,
                                        f16x8* qf) {
  constexpr int KSTEPS = D / 16;
  const int t = r0 + ln;
  const bool tv = t < p.T;
  const int tc = tv ? t : p.T - 1;
  const uint16_t* qcol = p.q_in + (long long)hq * D * p.T + tc;
  // All loads (q, then the lane's 32 cos/sin pairs) are issued before any
  // of them is used: one memory round trip.  Interleaved pairs beyond
  // rope_dim read a clamped (valid) table entry and are not applied.
  uint16_t xb[KSTEPS][8];
#pragma unroll
  for (int k = 0; k < KSTEPS; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) xb[k][e] = qcol[(long long)(16 * k + 8 * hh + e) * p.T];
  const bool half_split = p.rope_style == HL_ROPE_HALF_SPLIT;  // then rope_dim == D
  float2 cs[KSTEPS / 2][8];
  if (p.do_rope) {
    const float2* tab = p.rope_tab + tc;
    const int last_pair = p.rope_dim / 2 - 1;
#pragma unroll
    for (int k = 0; k < KSTEPS / 2; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // half-split: pair 16k+8hh+e (k < KSTEPS/2); interleaved: pair
        // (16kk+8hh+ee)/2 for kk = 2k + e/4 (the lane's even dims, in order)
        const int kk = 2 * k + (e >> 2), ee = 2 * (e & 3);
        const int i = half_split ? 16 * k + 8 * hh + e : min((16 * kk + 8 * hh + ee) / 2, last_pair);
        cs[k][e] = tab[(long long)i * p.T];
      }
  }
  float x[KSTEPS][8];
#pragma unroll
  for (int k = 0; k < KSTEPS; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) x[k][e] = from_bits<QDT>(xb[k][e]);
  if (p.q_norm_w) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < KSTEPS; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[k][e] * x[k][e];
    ss += __shfl_xor(ss, 32, 64);
    const float inv = 1.0f / sqrtf(ss / (float)D + p.eps);
#pragma unroll
    for (int k = 0; k < KSTEPS; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[k][e] = x[k][e] * inv * p.q_norm_w[16 * k + 8 * hh + e];
  }
  if (p.do_rope) {
    if (half_split) {
#pragma unroll
      for (int k = 0; k < KSTEPS / 2; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float2 c = cs[k][e];
          const float v0 = x[k][e], v1 = x[k + KSTEPS / 2][e];
          x[k][e] = v0 * c.x - v1 * c.y;
          x[k + KSTEPS / 2][e] = v0 * c.y + v1 * c.x;
        }
    } else {
#pragma unroll
      for (int k = 0; k < KSTEPS; ++k)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const int d = 16 * k + 8 * hh + e;
          if (d < p.rope_dim) {
            const float2 c = cs[k >> 1][4 * (k & 1) + e / 2];
            const float v0 = x[k][e], v1 = x[k][e + 1];
            x[k][e] = v0 * c.x - v1 * c.y;
            x[k][e + 1] = v0 * c.y + v1 * c.x;
          }
        }
    }
  }
  float qmax = 0.f;  // a Q operand value beyond fp16's range goes to the range record
#pragma unroll
  for (int k = 0; k < KSTEPS; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float y = tv ? x[k][e] * p.qscale : 0.f;
      qmax = fmaxf(qmax, fabsf(y));
      qf[k][e] = (_Float16)y;
    }
  if (qmax >= kF16Inf && p.range_flag) range_flag_set(p.range_flag);
}

// Ping-pong flash kernel.  A workgroup has 8 waves, two per SIMD (waves w
// and w + 4 share SIMD w % 4).  The waves run in two groups one phase apart
// (barrier between phases): while group 0 issues MFMAs (the previous tile's
// P.V and this tile's S^T = K Q^T), group 1 runs a softmax on the vector
// ALUs, and the next phase swaps the roles, so each SIMD keeps its matrix
// core and its vector ALU busy with the two waves' independent work.
//
// Wave w owns 32 query rows of one head: head w % nh of the workgroup's nh
// heads (one GQA group shares the K/V tiles), row block w / nh.  Per wave:
//   S^T[j][t] = K[j][:] . Q^T[:][t]     (v_mfma_f32_32x32x16_f16, K from LDS,
//                                        Q^T in registers; the accumulators
//                                        start at -m_run: scores arrive
//                                        relative to the row's reference max)
//   softmax over j for each row t (row t = lane % 32: in-lane plus one xor-32
//                                        exchange)
//   O^T[d][t] += V^T[d][j] . P^T[j][t]  (V from LDS, P^T straight from the
//                                        S^T registers as fp16)
// The O^T formulation keeps each row's rescale factor a per-lane scalar.
// K and V tiles go global -> LDS with direct (VGPR-free) copies into three
// K and three V stages, requested three phases before their matrix steps.  LDS rows
// are stored with their 16-byte chunks XOR-swizzled (K by the row, V by the
// row / 2) so that each fragment read's 16-lane groups hit distinct banks.
template <int D, int ODT, int QIN>
__global__ __launch_bounds__(512) void prefill_mfma_kernel(MfmaPrefillParams p) {
  constexpr int KSTEPS = D / 16;    // QK^T k-steps
  constexpr int DB = D / 32;        // 32-dim blocks of O^T
  constexpr int KCPR = D / 8;       // 16-byte chunks per K row (key j: D dims)
  constexpr int VCPR = BN / 8;      // 16-byte chunks per V row (dim d: BN keys)
  constexpr int KT = BN * D;        // K stage elements
  constexpr int VT = D * BN;        // V stage elements
  constexpr int KI = KT / 8 / 64 / 8;  // direct copies per wave per tile (K)
  constexpr int VI = VT / 8 / 64 / 8;  // (V)
  // Three K and three V stages, each tile copied one phase before the
  // softmax step that precedes its first matrix step: that softmax step
  // reads the first K fragments of the next matrix step, which then starts
  // with operands in registers instead of waiting on LDS.  (Prefetching the
  // first V fragments as well needs 16 more VGPRs than the kernel has.)
  constexpr int NS = 3;
  __shared__ __attribute__((aligned(1024))) uint16_t lds[NS * KT + NS * VT];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches
  const int grp = wave >> 2;                                  // 0 leads, 1 lags one phase
  const int hh = lane >> 5, ln = lane & 31;

  // Work item: heaviest (last) query blocks first; within a query block the
  // kv head varies fastest, so with the hardware's round-robin of workgroups
  // over the 8 XCDs a given kv head keeps landing on the same XCD (and L2)
  // whenever Hkv * head groups is a multiple of 8.
  const int per_q = p.n_head_kv * p.n_hgrp;
  const int item = blockIdx.x;
  const int qblk = p.n_qblk - 1 - item / per_q;
  const int kvh = (item % per_q) / p.n_hgrp;
  const int hgrp = (item % per_q) % p.n_hgrp;
  const int hq = kvh * p.group + hgrp * p.nh + (wave % p.nh);
  const int r0 = qblk * p.rows_wg + (wave / p.nh) * QR;  // this wave's first row
  const int wg_last_row = min(p.T - 1, qblk * p.rows_wg + p.rows_wg - 1);
  const int n_tiles = wg_last_row / BN + 1;
  const bool live = r0 < p.T;
  const int wave_tiles = live ? min(n_tiles, (r0 + QR - 1) / BN + 1) : 0;

  const uint16_t* kbase = p.kt + (long long)kvh * p.Tp * D;
  const uint16_t* vbase = p.vt + (long long)kvh * D * p.Tp;
  uint16_t* const kst0 = lds;
  uint16_t* const vst0 = lds + NS * KT;

  // Tile j -> its stage: every wave copies KI (K) or VI (V) 1 KB blocks.
  auto request_k = [&](int j) {
    uint16_t* st = kst0 + (j % NS) * KT;
#pragma unroll
    for (int r = 0; r < KI; ++r) {
      const int blk = wave * KI + r;            // 1 KB block of the K stage
      const int row = blk * (64 / KCPR) + lane / KCPR;
      const int slot = lane % KCPR;
      const int c = slot ^ (row % KCPR);
      copy16_to_lds(kbase + (long long)(j * BN + row) * D + 8 * c, st + blk * 512);
    }
  };
  auto request_v = [&](int j) {
    uint16_t* st = vst0 + (j % NS) * VT;
#pragma unroll
    for (int r = 0; r < VI; ++r) {
      const int blk = wave * VI + r;            // 1 KB block of the V stage
      const int d = blk * (64 / VCPR) + lane / VCPR;
      const int slot = lane % VCPR;
      const int c = slot ^ ((d >> 1) % VCPR);
      copy16_to_lds(vbase + (long long)d * p.Tp + j * BN + 8 * c, st + blk * 512);
    }
  };

  request_k(0);
  if (n_tiles > 1) request_k(1);
  request_v(0);

  // Q^T operand: lane holds q[t = r0 + ln][16*k + 8*hh .. +7]
  f16x8 qf[KSTEPS];
  if constexpr (QIN != 0) {
    build_q<D, QIN>(p, hq, r0, ln, hh, qf);
  } else {
    const int t = min(r0 + ln, p.Tp - 1);
    const uint16_t* qrow = p.qt + ((long long)hq * p.Tp + t) * D;
#pragma unroll
    for (int k = 0; k < KSTEPS; ++k) qf[k] = *(const f16x8*)(qrow + 16 * k + 8 * hh);
  }

  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
  // Scores are kept relative to a per-row reference max m_run (log2 units):
  // the S^T accumulators start at -m_run (negm), so the exponentials take
  // the MFMA output as it is.  m_run starts at the first tile's max and only
  // moves when a tile's max exceeds it by more than kRescale.
  float m_run = 0.f, l_run = 0.f;
  f32x16 negm;
#pragma unroll
  for (int i = 0; i < 16; ++i) negm[i] = 0.f;
  const int t_abs = r0 + ln;

  // Per-lane LDS offsets (elements) of the fragments this lane reads.
  int koff[2], voff[DB];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) koff[mb] = (32 * mb + sigma_row(ln)) * D;
#pragma unroll
  for (int db = 0; db < DB; ++db) voff[db] = (32 * db + ln) * BN;
  const int kswz[2] = {(32 * 0 + sigma_row(ln)) % KCPR, (32 * 1 + sigma_row(ln)) % KCPR};
  // V rows are 128 bytes (32 banks) apart, so a fragment read's bank group
  // is (row parity, chunk): swizzling the chunk by (row >> 1) makes the 16
  // lanes served together (rows ln .. ln+15) hit 16 distinct groups.
  const int vswz = (ln >> 1) % VCPR;  // ((32*db + ln) >> 1) % 8 == (ln >> 1) % 8

  f32x16 s[2];   // S^T of the tile between its QK^T and its softmax
  f16x8 pf[4];   // P^T of the tile between its softmax and its P.V:
                 // k-step 2*mb + u holds keys 16(2mb+u) + 8hh + 0..7

  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): K tiles 0, 1 and V tile 0 landed for this wave
  __syncthreads();

  f16x8 kpre[2][2];  // first K fragments of the next matrix step
  // Matrix step m: P.V of tile m - 1, then S^T of tile m.
  auto matrix_step = [&](const int j) {
    // Fragments
    // are read one k-step ahead of their MFMAs and the steps are fenced,
    // so only two steps' fragments are live (the other wave of the SIMD
    // covers the LDS latency with its softmax).
    const bool do_pv = j >= 1 && j - 1 < wave_tiles, do_qk = j < wave_tiles;
    const uint16_t* vst = vst0 + ((j + NS - 1) % NS) * VT;
    const uint16_t* kst = kst0 + (j % NS) * KT;
    const bool pre_k = j >= 1;  // first K fragments prefetched by vector_step(j - 1)
    if (do_pv) {
      f16x8 va[2][DB];
#pragma unroll
      for (int db = 0; db < DB; ++db) va[0][db] = *(const f16x8*)(vst + voff[db] + 8 * (hh ^ vswz));
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (u + 1 < 4) {
#pragma unroll
          for (int db = 0; db < DB; ++db)
            va[(u + 1) & 1][db] = *(const f16x8*)(vst + voff[db] + 8 * ((2 * (u + 1) + hh) ^ vswz));
        }
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db] = mma32(va[u & 1][db], pf[u], o[db]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (do_qk) {
      // Two k-steps of K fragments in flight ahead of the MFMAs.
      f16x8 kf[3][2];
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
          kf[k][mb] = pre_k ? kpre[k][mb] : *(const f16x8*)(kst + koff[mb] + 8 * ((2 * k + hh) ^ kswz[mb]));
#pragma unroll
      for (int k = 0; k < KSTEPS; ++k) {
        if (k + 2 < KSTEPS) {
#pragma unroll
          for (int mb = 0; mb < 2; ++mb)
            kf[(k + 2) % 3][mb] = *(const f16x8*)(kst + koff[mb] + 8 * ((2 * (k + 2) + hh) ^ kswz[mb]));
        }
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) s[mb] = mma32(kf[k % 3][mb], qf[k], k == 0 ? negm : s[mb]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // Vector step: softmax of tile j.
  auto vector_step = [&](const int j) {
    if (j < 0 || j >= wave_tiles) return;
    const int j0 = j * BN;
    if (j0 + BN - 1 > r0) {  // causal mask: key j > row t -> -inf
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int a = i >> 2;
          const int key = j0 + 32 * mb + 16 * (a >> 1) + 8 * hh + 4 * (a & 1) + (i & 3);
          s[mb][i] = key > t_abs ? -INFINITY : s[mb][i];
        }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) mt = fmaxf(mt, s[mb][i]);
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    // Every row t < T has an unmasked key j0 <= t in each tile it visits;
    // rows >= T (padding) score their zero-padded q, so mt is finite.
    // The first tile sets the reference; later ones move it only when
    // their max exceeds it by more than kRescale (then o and l rescale).
    const bool grew = j == 0 || mt > kRescale;
    if (__builtin_amdgcn_ballot_w64(grew) != 0) {  // uniform, rare after the first tile
      const float dm = grew ? mt : 0.f;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) s[mb][i] -= dm;
      if (j > 0) {
        const float alpha = fast_exp2(-dm);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
      }
      m_run += dm;
#pragma unroll
      for (int i = 0; i < 16; ++i) negm[i] = -m_run;
    }
    // Row sum of the tile in fp32 from the unrounded exponentials, four
    // independent chains; P itself is rounded to fp16 once (RNE, packed)
    // for the P.V MFMA.  (fp16 dot products against (1, 1) would sum the
    // rounded values in fewer instructions, but their results wait on the
    // matrix pipeline while the other group's MFMAs run.)
    float ps[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const f32x2v ev = {fast_exp2(s[mb][8 * u + e]), fast_exp2(s[mb][8 * u + e + 1])};
          const f16x2 pr = __builtin_convertvector(ev, f16x2);
          pf[2 * mb + u][e] = pr[0];
          pf[2 * mb + u][e + 1] = pr[1];
          ps[(e / 2) & 3] += ev.x + ev.y;
        }
    l_run += (ps[0] + ps[1]) + (ps[2] + ps[3]);
    // First K fragments of matrix step j + 1 (K(j+1), k-steps 0 and 1; the
    // tile is visible since the previous barrier).
    if (j + 1 < wave_tiles) {
      const uint16_t* kst = kst0 + ((j + 1) % NS) * KT;
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) kpre[k][mb] = *(const f16x8*)(kst + koff[mb] + 8 * ((2 * k + hh) ^ kswz[mb]));
    }
  };
  // Phase 2m takes K(m+2) into the stage of K(m-1) and V(m+1) into that of
  // V(m-2), whose last reads were in phase 2m-1.  After each odd phase every
  // wave's copies have landed and the barrier publishes them: K(m+2) and
  // V(m+1) are visible from phase 2m+2, a phase before the matrix steps
  // that use them, when the preceding softmax step prefetches from K.
  auto copies = [&](const int m) {
    if (m + 2 < n_tiles) request_k(m + 2);
    if (m + 1 < n_tiles) request_v(m + 1);
  };
  // Group 0 runs matrix step m in phase 2m and vector step m in phase 2m+1;
  // group 1 runs vector step m-1 in phase 2m and matrix step m in 2m+1.
  // Both loops pass the same barriers.
  if (grp == 0) {
    for (int m = 0; m <= n_tiles; ++m) {
      copies(m);
      __builtin_amdgcn_s_setprio(1);  // MFMAs issue ahead of the other group's VALU work
      matrix_step(m);
      __builtin_amdgcn_s_setprio(0);
      __syncthreads();
      vector_step(m);
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
    }
  } else {
    for (int m = 0; m <= n_tiles; ++m) {
      copies(m);
      vector_step(m - 1);
      __syncthreads();
      __builtin_amdgcn_s_setprio(1);  // MFMAs issue ahead of the other group's VALU work
      matrix_step(m);
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
    }
  }

  if (!live) return;
  const float l = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = 1.0f / l;
  if (t_abs < p.T) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = 32 * db + 8 * (i >> 2) + 4 * hh + (i & 3);
        store_elem<ODT>(p.out, ((long long)hq * D + d) * p.T + t_abs, o[db][i] * inv);
      }
  }
}

hipError_t prefill_mfma_launch(const PrefillLaunch& a, hipStream_t stream) {
  MfmaPrefillParams p;
  p.qt = a.qt;
  p.kt = a.kt;
  p.vt = a.vt;
  p.out = a.out;
  p.n_head = a.n_head;
  p.n_head_kv = a.n_head_kv;
  p.group = a.n_head / a.n_head_kv;
  p.T = a.seq_len;
  p.Tp = a.t_pad;
  p.nh = (p.group % 4 == 0) ? 4 : ((p.group % 2 == 0) ? 2 : 1);
  p.rows_wg = QR * (8 / p.nh);
  p.n_qblk = (p.T + p.rows_wg - 1) / p.rows_wg;
  p.n_hgrp = p.group / p.nh;
  p.q_in = (const uint16_t*)a.q_in;
  p.q_norm_w = a.q_norm_w;
  p.eps = a.eps;
  p.qscale = a.scale_log2;
  p.do_rope = a.do_rope;
  p.rope_dim = a.rope_dim;
  p.rope_style = a.rope_style;
  p.rope_tab = a.rope_tab;
  p.range_flag = a.range_flag;
  const int qin = a.qt ? 0 : a.io_dtype;
  dim3 grid(a.n_head_kv * p.n_hgrp * p.n_qblk);
#define HL_PF(DD, OD, QI) hipLaunchKernelGGL((prefill_mfma_kernel<DD, OD, QI>), grid, dim3(512), 0, stream, p)
#define HL_PF_Q(DD, OD)                          \
  switch (qin) {                                 \
    case HL_F16: HL_PF(DD, OD, HL_F16); break;   \
    case HL_BF16: HL_PF(DD, OD, HL_BF16); break; \
    default: HL_PF(DD, OD, 0); break;            \
  }
  if (a.head_dim == 64) {
    if (a.out_dtype == HL_F16) HL_PF_Q(64, HL_F16)
    else if (a.out_dtype == HL_BF16) HL_PF_Q(64, HL_BF16)
    else HL_PF_Q(64, HL_F32)
  } else if (a.head_dim == 128) {
    if (a.out_dtype == HL_F16) HL_PF_Q(128, HL_F16)
    else if (a.out_dtype == HL_BF16) HL_PF_Q(128, HL_BF16)
    else HL_PF_Q(128, HL_F32)
  } else {
    return hipErrorInvalidValue;
  }
#undef HL_PF_Q
#undef HL_PF
  return hipGetLastError();
}

// ===========================================================================
// fp32 path on the matrix cores: v_mfma_f32_32x32x2_f32 (fp32 products and
// accumulation), 4 waves; wave w owns 32 query rows of one head of the
// workgroup's nh heads (one GQA group shares the K/V tiles), row block
// w / nh.  Per 64-key tile:
//   S^T[j][t] = K[j][:] . Q^T[:][t]   (A = K from LDS, B = q in registers,
//                                      pre-scaled by scale * log2 e)
//   online softmax over j for row t = lane % 32 (in-lane + one xor-32)
//   O^T[d][t] += V^T[d][j] . P^T[j][t] (A = V from LDS, B = P in registers)
// MFMA k-step ks pairs element 2ks + h with lane half h.  S^T output row
// m = 8a + 4h + e of key block mb is key 32mb + 8a + 2e + h, so output
// register 4a + e of lane half h is exactly the P^T operand of P.V k-step
// 16mb + 4a + e: P never leaves registers.  K rows are staged in LDS as
// [h][key][ks], V rows as [h][d][ks] (ks = the pair index), 16-byte chunks
// XOR-swizzled by the row: one 16-byte read gives four k-steps' operands.
// ===========================================================================
namespace {
__device__ __forceinline__ f32x16 mma32f(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
}  // namespace

size_t prefill_f32_split_bytes(int n_head_kv, int head_dim, int seq_len) {
  if (head_dim != 64 && head_dim != 128) return 0;
  return (size_t)n_head_kv * ((seq_len + 63) / 64) * (split_img_bytes(head_dim) + 4 * kSplitRecInts);
}

// FB: the gated fallback pass of an MFMA prefill (a grid of at most one
// workgroup per CU looping over the items, output in out_dtype); otherwise
// one item per workgroup and fp32 output, with no loop or gate in the code.
// X3: each step runs its two products as three fp16 MFMAs on a hi/lo split
// of every fp32 operand (hi hi + (hi lo + lo hi) 2^-11, to ~2^-21 of each
// product: within fp32 rounding of the dot products) instead of fp32 MFMAs,
// which the matrix cores run at 1/16 of the fp16 rate.  The operands are
// scaled by powers of two first (Q per row, K and V per 32-key half tile, P
// by 2^14 or less), so that every element within 2^27 of its set's largest
// keeps a normal fp16 hi part; the products are unscaled exactly.  K and V
// arrive split, from the prologue's per-tile images (two LDS sets, the next
// step's copied in during this one); Q is split per wave.  A step whose
// tiles (the prologue's flags) or the workgroup's Q (a vote before the first
// step) hold an inf or NaN runs the fp32 MFMAs on fp32 tiles loaded at that
// step.
template <int D, int KSPLIT, bool FB, bool X3 = false>
__global__ __launch_bounds__(256) void prefill_f32mfma_kernel(PrefillLaunch p, int nh) {
  constexpr int NW = 4;             // waves
  constexpr int KS = D / 2;         // S^T k-steps (pairs of head dims)
  constexpr int KC = KS / 4;        // 16-byte chunks per staged K row
  constexpr int DB = D / 32;        // 32-dim blocks of O^T
  constexpr int BN = 64;            // keys per tile
  constexpr int NL = D * BN / (64 * NW);  // K (and V) tile elements per thread and tile
  // KSPLIT key groups: wave w serves head w % nh and the key tiles
  // kq, kq + KSPLIT, ... (kq = w / nh); each step stages KSPLIT tiles.
  constexpr int SKN = 2 * BN * KS, SVN = 2 * D * 32;
  // X3: two sets of KSPLIT tiles, the next step's copied in while this
  // step's are read.
  constexpr int NBUF = X3 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) float sk[NBUF * KSPLIT * SKN];  // [buf][tile][h][key][ks]
  __shared__ __attribute__((aligned(16))) float sv[NBUF * KSPLIT * SVN];  // [buf][tile][h][d][ks]

  const int tid = threadIdx.x, lane = tid & 63;
  if constexpr (FB) {
    // Fallback pass of an MFMA prefill: runs only when the call's overflow
    // mark F equals the staged S; workgroup 0 then advances the generation
    // (G = S, which nothing else in this kernel reads) and records the outcome.
    __shared__ unsigned s_go;
    if (tid == 0) {
      unsigned* rec = p.fallback_record;
      const unsigned sg = rec[2];
      const unsigned go = rec[0] == sg;
      if (blockIdx.x == 0) {
        rec[1] = sg;
        rec[3] = go;
      }
      s_go = go;
    }
    __syncthreads();
    if (!s_go) return;
  }
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, hh = lane >> 5;
  const int T = p.seq_len;
  const int group = p.n_head / p.n_head_kv;
  // wave = (kq * RB + rb) * nh + head: key group kq, row block rb, head.
  const int RB = NW / (nh * KSPLIT);             // 32-row blocks per workgroup (1 when split)
  const int kq = wave / (nh * RB);
  const int rows_wg = 32 * RB;
  const int n_qblk = (T + rows_wg - 1) / rows_wg;
  const int n_hgrp = group / nh;
  const int per_q = p.n_head_kv * n_hgrp;
  // Each item's first barrier (before its LDS fill) waits for every wave's
  // previous item (fallback pass).
  auto run_item = [&](const int item) {
    // In the fallback's item loop the lane and wave ids are re-derived per
    // item behind an empty asm: otherwise the per-lane load offsets (32 per
    // K/V row set) are hoisted out of the loop and kept live across the
    // whole item, which pushes the kernel into scratch at head dim 128.
    int lane_i = lane, wave_i = wave, tid_i = tid;
    if constexpr (FB) {
      lane_i = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
      asm volatile("" : "+v"(lane_i), "+s"(wave_i));
      tid_i = wave_i * 64 + lane_i;
    }
    const int lane = lane_i, wave = wave_i, tid = tid_i;
    const int ln = lane & 31, hh = lane >> 5;
    const int qblk = n_qblk - 1 - item / per_q;  // heaviest query blocks first
    const int kvh = (item % per_q) / n_hgrp;
    const int hgrp = (item % per_q) % n_hgrp;
    const int hq = kvh * group + hgrp * nh + wave % nh;
    const int r0 = qblk * rows_wg + ((wave / nh) % RB) * 32;
    const int wg_last_row = min(T - 1, qblk * rows_wg + rows_wg - 1);
    const int n_tiles = wg_last_row / BN + 1;
    const int n_steps = (n_tiles + KSPLIT - 1) / KSPLIT;
    const int t_abs = r0 + ln;
    const bool live = r0 < T;

    const float* K = p.k + (long long)kvh * D * T;
    const float* V = p.v + (long long)kvh * D * T;
    // Swizzled 16-byte chunk of a staged fp32 row (rows 2D or 128 bytes long).
    auto kswz = [](int key) { return D == 64 ? (key >> 1) & 7 : key & 15; };
    auto vswz = [](int d) { return (d >> 1) & 7; };

    // fp32 K/V tiles: thread moves column lc (key j0 + lc) of rows
    // d = ld0 + 4k; the next step's tiles are loaded while the current ones
    // are computed.  X3: only a step that runs the fp32 MFMAs loads them, at
    // the step; the split tiles come from the images the prologue wrote,
    // copied straight into LDS one step ahead; the fp32 steps pass the
    // thread id through an empty asm, so that their
    // per-lane addresses are computed at the step instead of being hoisted
    // and kept live across the loop (which costs the split steps registers).
    float kr[KSPLIT][NL], vr[KSPLIT][NL];
    auto load_kv = [&](int step, int tid_) {
      const int lc = tid_ & 63, ld0 = tid_ >> 6;
#pragma unroll
      for (int u = 0; u < KSPLIT; ++u) {
        const int col = min((step * KSPLIT + u) * BN + lc, T - 1);
#pragma unroll
        for (int k = 0; k < NL; ++k) {
          kr[u][k] = K[(long long)(ld0 + NW * k) * T + col];
          vr[u][k] = V[(long long)(ld0 + NW * k) * T + col];
        }
      }
    };
    // Writes the loaded tiles to LDS set b in the fp32 layout (keys past T
    // as zeros).
    auto stage_f32 = [&](int step, int b, int tid_) {
      const int lc = tid_ & 63, ld0 = tid_ >> 6;
#pragma unroll
      for (int u = 0; u < KSPLIT; ++u) {
        const bool in = (step * KSPLIT + u) * BN + lc < T;
        float* tk = sk + (b * KSPLIT + u) * SKN;
        float* tv = sv + (b * KSPLIT + u) * SVN;
#pragma unroll
        for (int k = 0; k < NL; ++k) {
          const int d = ld0 + NW * k;
          const float kx = in ? kr[u][k] : 0.f, vx = in ? vr[u][k] : 0.f;
          // K: (h = d & 1, key = lc, ks = d >> 1); V: (h = lc & 1, d, ks = lc >> 1)
          const int ksk = d >> 1, ksv = lc >> 1;
          tk[((d & 1) * BN + lc) * KS + (((ksk >> 2) ^ kswz(lc)) << 2) + (ksk & 3)] = kx;
          tv[((lc & 1) * D + d) * 32 + (((ksv >> 2) ^ vswz(d)) << 2) + (ksv & 3)] = vx;
        }
      }
    };
    // X3: a tile's image into LDS set b, 1 KB per wave copy:
    // the K image into the set's K tile, the V image into its V tile.
    const int n_kt = (T + BN - 1) / BN;
    [[maybe_unused]] const char* img = (const char*)p.kv_img + (long long)kvh * n_kt * split_img_bytes(D);
    [[maybe_unused]] const int* meta = p.kv_meta + (long long)kvh * n_kt * kSplitRecInts;
    [[maybe_unused]] auto issue_copies = [&](int step, int b) {
#pragma unroll
      for (int u = 0; u < KSPLIT; ++u) {
        const int tl = step * KSPLIT + u;
        if (tl >= n_tiles) continue;
        const char* src = img + (long long)tl * split_img_bytes(D) + lane * 16;
        constexpr int NCH = split_img_bytes(D) / 1024, HALF = NCH / 2;
#pragma unroll
        for (int i = 0; i < NCH / NW; ++i) {
          const int ch = wave + NW * i;
          char* dst = ch < HALF ? (char*)(sk + (b * KSPLIT + u) * SKN) + ch * 1024
                                : (char*)(sv + (b * KSPLIT + u) * SVN) + (ch - HALF) * 1024;
          copy16_to_lds(src + ch * 1024, dst);
        }
      }
    };
    // X3: the step's tile records (any flag among its tiles; the shifts of
    // this wave's tile's two halves), loaded with the step's copies, a step
    // ahead.
    [[maybe_unused]] int m_bad = 0, m_shk0 = 0, m_shk1 = 0, m_shv0 = 0, m_shv1 = 0;
    [[maybe_unused]] auto load_meta = [&](int step) {
      m_bad = 0;
#pragma unroll
      for (int u = 0; u < KSPLIT; ++u) {
        const int tl = min(step * KSPLIT + u, n_tiles - 1);  // a tile past the workgroup's repeats one
        const int4 f = *(const int4*)(meta + tl * kSplitRecInts + 4);
        m_bad |= f.x | f.y | f.z | f.w;
      }
      const int4 sh = *(const int4*)(meta + min(step * KSPLIT + kq, n_tiles - 1) * kSplitRecInts);
      m_shk0 = sh.x;
      m_shk1 = sh.y;
      m_shv0 = sh.z;
      m_shv1 = sh.w;
    };
    if constexpr (X3) {
      issue_copies(0, 0);
      load_meta(0);
    } else {
      load_kv(0, tid);
    }

    // q operand: lane (ln, hh) holds q[t][2ks + hh] * scale * log2 e
    // (X3: loaded again in each fp32 step instead, so that the 2 x 32 or
    // 2 x 64 q registers of the two forms are not both live in the loop.)
    float qv[KS];
    auto load_qv = [&](int lane_) {
      const float* Q = p.q + (long long)hq * D * T;
      const int t = min(r0 + (lane_ & 31), T - 1), h_ = lane_ >> 5;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qv[ks] = Q[(long long)(2 * ks + h_) * T + t] * p.scale_log2;
    };
    if constexpr (!X3) load_qv(lane);
    // X3: lane (ln, hh) also holds q[t][16 ks + 8 hh + j] * scale * log2 e *
    // 2^sq as the fp16 hi/lo B operand of the S^T = K Q^T MFMAs, sq scaling
    // the row's largest element (over both lane halves) into [2^13, 2^14);
    // qbad: an inf or NaN among them.
    [[maybe_unused]] f16x8 qh[X3 ? D / 16 : 1], ql[X3 ? D / 16 : 1];
    [[maybe_unused]] bool qbad = false;
    [[maybe_unused]] int sq = 0;
    if constexpr (X3) {
      const float* Q = p.q + (long long)hq * D * T;
      const int t = min(t_abs, T - 1);
      float x[D / 16][8];
      uint32_t mq = 0u;
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          x[ks][j] = Q[(long long)(16 * ks + 8 * hh + j) * T + t] * p.scale_log2;
          mq = max(mq, __float_as_uint(x[ks][j]) & 0x7FFFFFFFu);
        }
      mq = max(mq, (uint32_t)__shfl_xor((int)mq, 32, 64));
      qbad = live && mq >= kInfBits;
      sq = qbad ? 0 : split_shift(mq);
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[ks][j] = __builtin_amdgcn_ldexpf(x[ks][j], sq);
        split_f16x8(x[ks], qh[ks], ql[ks]);
      }
    }

    f32x16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
    // X3: each wave's Q flag, read after the first step's barrier.
    [[maybe_unused]] __shared__ uint32_t s_qbad[NW];
    if constexpr (X3)
      if (lane == 0) s_qbad[wave] = __builtin_amdgcn_ballot_w64(qbad) != 0;
    float m_run = -INFINITY, l_run = 0.f;

    for (int step = 0; step < n_steps; ++step) {
      // The previous step's sk / sv reads are done.
      bool x3 = false;
      [[maybe_unused]] int shk0 = 0, shk1 = 0, shv0 = 0, shv1 = 0;
      const int b = X3 ? (step & 1) : 0;  // LDS set of this step
      if constexpr (X3) {
        // This wave's copies of the step's images have landed; after the
        // barrier every wave's have, and the other set's readers (the previous
        // step) are done, so the next step's copies may start.
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        // Split steps unless a tile of the step or the workgroup's Q holds an
        // inf or NaN (the split kernel's flag per tile, the Q vote).
        x3 = (m_bad | s_qbad[0] | s_qbad[1] | s_qbad[2] | s_qbad[3]) == 0;
        shk0 = m_shk0;
        shk1 = m_shk1;
        shv0 = m_shv0;
        shv1 = m_shv1;
        // A wave that runs this step's split products issues the next step's
        // copies behind its first matrix instructions (below); the others now.
        if (!(x3 && live && (step * KSPLIT + kq) * BN <= r0 + 31)) {
          if (step + 1 < n_steps) issue_copies(step + 1, b ^ 1);
          load_meta(min(step + 1, n_steps - 1));  // unconditional: no join that waits for it
        }
        if (!x3) {
          // fp32 MFMA step: the fp32 tiles replace this set's images
          int tid_ = tid;
          asm volatile("" : "+v"(tid_));
          load_kv(step, tid_);
          stage_f32(step, b, tid_);
          __syncthreads();
        }
      } else {
        __syncthreads();
        stage_f32(step, 0, tid);
        if (step + 1 < n_steps) load_kv(step + 1, tid);
        __syncthreads();
      }
      const int j0 = (step * KSPLIT + kq) * BN;
      if (!live || j0 > r0 + 31) continue;  // wave-uniform: no key of this tile is visible
      const float* tk = sk + (b * KSPLIT + kq) * SKN;
      const float* tv = sv + (b * KSPLIT + kq) * SVN;
      if constexpr (X3) {
        if (x3) {
          const uint16_t* kh = (const uint16_t*)tk;
          const uint16_t* kl = kh + BN * D;
          const uint16_t* vh = (const uint16_t*)tv;
          const uint16_t* vl = vh + D * BN;
          // S^T = K Q^T: A row m = key 32 mb + sigma(m) (the bf16 flash kernel's
          // permutation: P^T then feeds the P V MFMAs as it is).
          f32x16 s[2];
#pragma unroll
          for (int mb = 0; mb < 2; ++mb) {
            const int key = 32 * mb + sigma_row(ln);
            f32x16 s1, s2;
#pragma unroll
            for (int i = 0; i < 16; ++i) s1[i] = s2[i] = 0.f;
#pragma unroll
            for (int ks = 0; ks < D / 16; ++ks) {
              const int pos = key * D + 8 * ((2 * ks + hh) ^ (key % (D / 8)));
              const f16x8 ah = *(const f16x8*)(kh + pos), al = *(const f16x8*)(kl + pos);
              s1 = mma32(ah, qh[ks], s1);
              s2 = mma32(ah, ql[ks], s2);
              s2 = mma32(al, qh[ks], s2);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i)
              s[mb][i] = __builtin_amdgcn_ldexpf(s1[i] + s2[i] * 0x1p-11f, -(sq + (mb ? shk1 : shk0)));
            if (mb == 0) {
              if (step + 1 < n_steps) issue_copies(step + 1, b ^ 1);
              load_meta(min(step + 1, n_steps - 1));
            }
          }
          // Register i = 4a + e of lane half hh in block mb: key
          // j0 + 32 mb + 16 (a >> 1) + 8 hh + 4 (a & 1) + e.  A tile before
          // the row block's first row and inside T needs no mask (wave-uniform).
          float mt = -INFINITY;
          if (j0 + BN - 1 <= r0 && j0 + BN <= T) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
              for (int i = 0; i < 16; ++i) mt = fmaxf(mt, s[mb][i]);
          } else {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
              for (int i = 0; i < 16; ++i) {
                const int a = i >> 2;
                const int key = j0 + 32 * mb + 16 * (a >> 1) + 8 * hh + 4 * (a & 1) + (i & 3);
                s[mb][i] = (key <= t_abs && key < T) ? s[mb][i] : -INFINITY;
                mt = fmaxf(mt, s[mb][i]);
              }
          }
          mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
          const float mn = fmaxf(m_run, mt);
          const float alpha = fast_exp2(m_run - mn);
          m_run = mn;
          float ps = 0.f;
#pragma unroll
          for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              s[mb][i] = fast_exp2(s[mb][i] - mn);
              ps += s[mb][i];
            }
          l_run = l_run * alpha + ps;
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
          // O^T += V^T P^T, k-step u = keys 16 u + 8 hh + j of this lane's row
          // (key half u / 2), into this tile's own accumulators, unscaled into
          // o.  V of half h is scaled by 2^shv_h; P of that half by
          // 2^(14 + shv_min - shv_h), so that every product carries
          // 2^(14 + shv_min): P * 2^14 in the half with the larger values (its
          // hi parts normal down to P = 2^-28), less in the other.
          const int shv_min = min(shv0, shv1);
          f16x8 ph[4], pl[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int pe = 14 + shv_min - ((u >> 1) ? shv1 : shv0);
            float x[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
              x[j] = __builtin_amdgcn_ldexpf(s[u >> 1][4 * (2 * (u & 1) + (j >> 2)) + (j & 3)], pe);
            split_f16x8(x, ph[u], pl[u]);
          }
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const int d = 32 * db + ln;
            f32x16 t1, t2;
#pragma unroll
            for (int i = 0; i < 16; ++i) t1[i] = t2[i] = 0.f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int pos = d * BN + 8 * ((2 * u + hh) ^ ((d >> 1) & 7));
              const f16x8 vh8 = *(const f16x8*)(vh + pos), vl8 = *(const f16x8*)(vl + pos);
              t1 = mma32(vh8, ph[u], t1);
              t2 = mma32(vh8, pl[u], t2);
              t2 = mma32(vl8, ph[u], t2);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] += __builtin_amdgcn_ldexpf(t1[i] + t2[i] * 0x1p-11f, -(shv_min + 14));
          }
          continue;
        }
      }

      if constexpr (X3) {
        int lane_ = lane;
        asm volatile("" : "+v"(lane_));
        load_qv(lane_);
      }
      f32x16 s[2];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const int m = ln;  // A operand row = key 32mb + 8a + 2e + h for m = 8a + 4h + e
        const int key = 32 * mb + 8 * (m >> 3) + 2 * (m & 3) + ((m >> 2) & 1);
        const float* row = tk + (hh * BN + key) * KS;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[mb][i] = 0.f;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          const f32x4 kf = *(const f32x4*)(row + ((c ^ kswz(key)) << 2));
#pragma unroll
          for (int e = 0; e < 4; ++e) s[mb] = mma32f(kf[e], qv[4 * c + e], s[mb]);
        }
      }
      // Causal mask and keys beyond T: output register i = 4a + e of lane half
      // hh in block mb is key j0 + 32mb + 8a + 2e + hh.
      float mt = -INFINITY;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = j0 + 32 * mb + 8 * (i >> 2) + 2 * (i & 3) + hh;
          s[mb][i] = (key <= t_abs && key < T) ? s[mb][i] : -INFINITY;
          mt = fmaxf(mt, s[mb][i]);
        }
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      // Finite: a visible tile starts at or before the row block (tiles are 64
      // keys, row blocks 32 rows, both aligned), so every row sees key j0.
      const float mn = fmaxf(m_run, mt);
      const float alpha = fast_exp2(m_run - mn);
      m_run = mn;
      float ps = 0.f;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          s[mb][i] = fast_exp2(s[mb][i] - mn);
          ps += s[mb][i];
        }
      l_run = l_run * alpha + ps;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
      // O^T += V^T P^T: k-step ks = 16mb + i pairs keys 2ks + h.
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int d = 32 * db + ln;
        const float* row = tv + (hh * D + d) * 32;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const f32x4 vf = *(const f32x4*)(row + ((c ^ vswz(d)) << 2));
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int ks = 4 * c + e;
            o[db] = mma32f(vf[e], s[ks >> 4][ks & 15], o[db]);
          }
        }
      }
    }

    float l = l_run + __shfl_xor(l_run, 32, 64);
    if constexpr (KSPLIT > 1) {
      // Key groups 1.. hand (m, l, o) to group 0 through LDS (the tiles are
      // dead); a group that saw no tile has m = -inf and weight 0.
      __syncthreads();
      // Slots: the waves of key groups 1.., slot = wave - nh (the launch uses
      // the split only with one row block per workgroup, RB = 1).
      constexpr int NSLOT = NW - NW / KSPLIT;
      float* xm = sk;                  // [slot][lane] m
      float* xl = xm + NSLOT * 64;     // [slot][lane] l
      float* xo = xl + NSLOT * 64;     // [slot][db*16 + i][lane] o
      static_assert(NSLOT * 64 * (2 + 16 * DB) <= KSPLIT * SKN, "merge buffers fit the K tiles");
      if (kq > 0) {
        const int sl = wave - nh;
        xm[sl * 64 + lane] = m_run;
        xl[sl * 64 + lane] = l;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) xo[(sl * 16 * DB + db * 16 + i) * 64 + lane] = o[db][i];
      }
      __syncthreads();
      if (kq > 0) return;  // key groups 1.. are done with this item
      // O^T layout: every element this lane holds belongs to its own query
      // row t_abs, so the merge factors are per-lane scalars.
      float mall = m_run;
#pragma unroll
      for (int q = 1; q < KSPLIT; ++q) mall = fmaxf(mall, xm[(wave + (q - 1) * nh) * 64 + lane]);
      const float a0 = fast_exp2(m_run - mall);
      float aq[KSPLIT];
      l *= a0;
#pragma unroll
      for (int q = 1; q < KSPLIT; ++q) {
        const int sl = wave + (q - 1) * nh;  // slot of this row block's key group q
        aq[q] = fast_exp2(xm[sl * 64 + lane] - mall);  // 0 for a group with no tile
        l += aq[q] * xl[sl * 64 + lane];
      }
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float v = o[db][i] * a0;
#pragma unroll
          for (int q = 1; q < KSPLIT; ++q)
            v += aq[q] * xo[((wave + (q - 1) * nh) * 16 * DB + db * 16 + i) * 64 + lane];
          o[db][i] = v;
        }
    }
    if (!live) return;
    const float inv = 1.0f / l;
    if (t_abs < T) {
      // fp32 output, or fp16 / bf16 when this is the fallback of an MFMA prefill
      const long long ob = (long long)hq * D * T + t_abs;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int d = 32 * db + 8 * (i >> 2) + 4 * hh + (i & 3);
          const float y = o[db][i] * inv;
          if (FB && p.out_dtype == HL_F16) store_elem<HL_F16>(p.out, ob + (long long)d * T, y);
          else if (FB && p.out_dtype == HL_BF16) store_elem<HL_BF16>(p.out, ob + (long long)d * T, y);
          else ((float*)p.out)[ob + (long long)d * T] = y;
        }
    }
  };
  if constexpr (FB) {
    const int n_items = per_q * n_qblk;
    for (int item = blockIdx.x; item < n_items; item += gridDim.x) run_item(item);
  } else {
    run_item(blockIdx.x);
  }
}

hipError_t prefill_f32_launch(const PrefillLaunch& p, hipStream_t stream) {
  const int group = p.n_head / p.n_head_kv;
  int nh = (group % 4 == 0) ? 4 : ((group % 2 == 0) ? 2 : 1);  // heads per workgroup
  auto grid_of = [&](int nh_, int ks) {
    const int rows_wg = 32 * (4 / (nh_ * ks));
    return p.n_head_kv * (group / nh_) * ((p.seq_len + rows_wg - 1) / rows_wg);
  };
  // Split each row block's keys over two wave groups (two heads per
  // workgroup) when four-head workgroups would leave CUs idle: twice the
  // workgroups, half the longest causal walk.
  // (A four-way split, one head per workgroup, measured 9% slower at c2.)
  const int ksp = (nh >= 2 && grid_of(nh, 1) < 256 && p.head_dim == 64) ? 2 : 1;
  if (ksp > 1) nh = 2;
  const int items = grid_of(nh, ksp);
  const dim3 grid(p.fallback_record ? std::min(items, cu_count()) : items);
  // the X3 kernels read the split images the prologue wrote
  if (!p.fallback_record && (!p.kv_img || !p.kv_meta)) return hipErrorInvalidValue;
#define HL_F32K(DD, KS)                                                                              \
  if (p.fallback_record) hipLaunchKernelGGL((prefill_f32mfma_kernel<DD, KS, true>), grid, dim3(256), 0, stream, p, nh); \
  else hipLaunchKernelGGL((prefill_f32mfma_kernel<DD, KS, false, true>), grid, dim3(256), 0, stream, p, nh)
  // The split-operand steps (X3) except in the fallback pass of an MFMA
  // prefill, which keeps the fp32 MFMAs.
  switch (p.head_dim) {
    case 64:
      if (ksp == 2) HL_F32K(64, 2);
      else HL_F32K(64, 1);
      break;
    case 128: HL_F32K(128, 1); break;
    default: return hipErrorInvalidValue;
  }
#undef HL_F32K
  return hipGetLastError();
}

}  // namespace hl
