// qkNorm, RoPE and KV-cache store kernels for gfx950.
//
// Reference kernels replaced (backends/naive.nim):
//   qkNormKernel / qkNormPrefillKernel          :2887-2971
//   ropeAtPosKernel / ropeQKDecodeKernel /
//   ropeAtPosThetaKernel                        :3006-3144
//   fusedRopeStoreKVKernel                      :3149-3223
//   storeKVKernel / storeKVPairKernel           :3228-3285
// The reference launches one of these per tensor per layer (up to six per
// attention layer); here one launch covers every head vector of a decode
// step (headvec_kernel) or every (32-token tile, group of heads) of a prefill
// (prologue_kernel), with the cache write and the conversion to the MFMA
// operand layout done while the data is in registers/LDS.
//
// Formulas kept from the reference:
//   RMSNorm   x * (1/sqrtf(sum(x^2)/D + eps)) * w[d]          (:2910, :2915)
//   RoPE      angle = float(pos) * theta[i];                    (:3065-3073)
//             (v0, v1) -> (v0*c - v1*s, v0*s + v1*c)
//             half-split pairs (i, i+rope_dim/2), or interleaved (2i, 2i+1)
//             as in tensor.nim:156-166; dims >= rope_dim pass through
//   theta[i]  powf(1/base, 2i/rope_dim) on the host (:3850-3861), passed to
//             the kernel by value.
#include "common.h"
#include "headvec.h"
#include "launch.h"

namespace hl {

// ---------------------------------------------------------------------------
// Decode side: one wave per head vector of the new token.
// blockIdx.x in [0, Hq): q heads; [Hq, Hq+Hkv): k heads; [Hq+Hkv, Hq+2Hkv): v.
// ---------------------------------------------------------------------------
template <int KDT>
__global__ __launch_bounds__(64) void headvec_kernel(HeadVecOp op) {
  __shared__ float sx[HL_MAX_HEAD_DIM];
  const int lane = threadIdx.x;
  const int b = blockIdx.y;
  const int D = op.head_dim;
  int hv = blockIdx.x;
  int kind;  // 0 q, 1 k, 2 v
  if (hv < op.n_head_q) {
    kind = 0;
  } else if (hv < op.n_head_q + op.n_head_kv) {
    kind = 1;
    hv -= op.n_head_q;
  } else {
    kind = 2;
    hv -= op.n_head_q + op.n_head_kv;
  }
  float* x = nullptr;
  const float* xin = nullptr;
  const float* nw = nullptr;
  int rope = 0;
  void* cache = nullptr;
  if (kind == 0) {
    if (!op.q) return;
    x = op.q + ((long long)b * op.n_head_q + hv) * D;
    xin = x;
    nw = op.q_norm_w;
    rope = op.rope_q;
  } else if (kind == 1) {
    if (!op.k) return;
    x = op.k + ((long long)b * op.n_head_kv + hv) * D;
    xin = x;
    nw = op.k_norm_w;
    rope = op.rope_k;
    cache = op.k_cache;
  } else {
    if (!op.v) return;
    xin = op.v + ((long long)b * op.n_head_kv + hv) * D;
    cache = op.v_cache;
  }

  for (int d = lane; d < D; d += 64) sx[d] = xin[d];
  wave_lds_sync();
  const int pos = op.positions ? op.positions[b] : op.pos;
  headvec_norm_rope(sx, D, lane, nw, op.eps, (rope && op.do_rope) ? op.rope_dim : 0, op.rope_style,
                    op.theta, pos);
  if (x && (nw || (rope && op.do_rope)))
    for (int d = lane; d < D; d += 64) x[d] = sx[d];
  if (cache) {
    const long long base = (long long)b * op.batch_stride + (long long)hv * D * op.max_len;
    for (int d = lane; d < D; d += 64) {
      const long long at = op.kv_layout == HL_KV_PAGED32
                               ? kv_paged_off(op.block_table, op.bps, b, op.n_head_kv, hv, D, d, pos)
                               : base + kv_off(op.kv_layout, d, pos, D, op.max_len);
      store_elem<KDT>(cache, at, sx[d]);
    }
  }
}

hipError_t headvec_launch(const HeadVecOp& op, hipStream_t stream) {
  dim3 grid(op.n_head_q + 2 * op.n_head_kv, op.batch);
  switch (op.kv_dtype) {
    case HL_F32: hipLaunchKernelGGL(headvec_kernel<HL_F32>, grid, dim3(64), 0, stream, op); break;
    case HL_F16: hipLaunchKernelGGL(headvec_kernel<HL_F16>, grid, dim3(64), 0, stream, op); break;
    case HL_FP8: hipLaunchKernelGGL(headvec_kernel<HL_FP8>, grid, dim3(64), 0, stream, op); break;
    default: hipLaunchKernelGGL(headvec_kernel<HL_BF16>, grid, dim3(64), 0, stream, op); break;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Prefill side: one workgroup per (32-token tile, group of kHPG head vectors)
// of col-major [H*D, T] activations.  Head vectors are numbered q heads, then
// k heads, then v heads.  The workgroup evaluates cos/sin of its 32 positions
// once (an LDS table of rope_dim/2 x 32 entries) and reuses it for every q/k
// head of its group: RoPE's trigonometry is per (position, pair), not per
// head, and with angles up to ~T rad it is the costly part of this kernel.
// ---------------------------------------------------------------------------
constexpr int kPT = 32;   // tokens per tile
constexpr int kHPG = 8;   // most head vectors per workgroup
constexpr int kTabHalf = 64;  // largest rope_dim/2 served from the LDS table

// 8 consecutive elements [t, t+8) of one activation row as fp32; t >= lim -> 0.
template <int DT>
__device__ __forceinline__ void load_row8_f32(const void* base, long long off, int t, int lim,
                                              float* x) {
  static_assert(DT != HL_FP8, "activations are fp32/fp16/bf16");
  const int esz = DT == HL_F32 ? 4 : 2;
  if (t + 8 <= lim && (((uintptr_t)base + (uintptr_t)off * esz) & 15) == 0) {
    if constexpr (DT == HL_F32) {
      const f32x4 a = *(const f32x4*)((const float*)base + off);
      const f32x4 b = *(const f32x4*)((const float*)base + off + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = a[e];
        x[e + 4] = b[e];
      }
    } else {
      const u16x8 v = *(const u16x8*)((const uint16_t*)base + off);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = from_bits<DT>(v[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (t + e < lim) ? load_elem<DT>(base, off + e) : 0.f;
  }
}

// Stores 8 consecutive elements [t, t+8) of one row; elements >= lim skipped.
// Vector stores need 16-byte alignment (8 bytes for fp8).
template <int DT>
__device__ __forceinline__ void store_row8(void* base, long long off, int t, int lim,
                                           const float* x) {
  constexpr int esz = elem_bytes<DT>();
  constexpr uintptr_t amask = DT == HL_FP8 ? 7 : 15;
  if (t + 8 <= lim && (((uintptr_t)base + (uintptr_t)off * esz) & amask) == 0) {
    if constexpr (DT == HL_F32) {
      *(f32x4*)((float*)base + off) = f32x4{x[0], x[1], x[2], x[3]};
      *(f32x4*)((float*)base + off + 4) = f32x4{x[4], x[5], x[6], x[7]};
    } else if constexpr (DT == HL_FP8) {
      uint32_t w[2] = {0u, 0u};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = x[e];
        __asm__ volatile("" : "+v"(v));  // round the fp32 value, as store_elem does
        w[e >> 2] |= (uint32_t)f32_to_e4m3(v) << (8 * (e & 3));
      }
      typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
      *(u32x2v*)((uint8_t*)base + off) = u32x2v{w[0], w[1]};
    } else {
      u16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = to_bits<DT>(x[e]);
      *(u16x8*)((uint16_t*)base + off) = v;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (t + e < lim) store_elem<DT>(base, off + e, x[e]);
  }
}

// Where a prefill's cache columns go: one sequence, kv head h, row d.
struct CacheMap {
  int layout, D, max_len, n_head_kv;
  const int* table;  // paged: the sequence's pages
};
__device__ __forceinline__ long long cache_off(const CacheMap& m, int h, int d, int t) {
  if (m.layout == HL_KV_PAGED32) return kv_paged_off(m.table, 0, 0, m.n_head_kv, h, m.D, d, t);
  return (long long)h * m.D * m.max_len + kv_off(m.layout, d, t, m.D, m.max_len);
}

// Cache columns pos .. pos+7 of row d of kv head h, the values of tokens
// t .. t+7 (t + e < lim stored): one vector store when the 8 columns are
// contiguous and aligned in the layout (tiled and paged caches: when they
// stay inside one 32-column tile), else element by element.
template <int DT>
__device__ __forceinline__ void store_cache8(void* cache, const CacheMap& m, int h, int d, int pos,
                                             int t, int lim, const float* x) {
  if (m.layout != HL_KV_COLMAJOR && (pos & 31) > 24) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (t + e < lim) store_elem<DT>(cache, cache_off(m, h, d, pos + e), x[e]);
  } else {
    store_row8<DT>(cache, cache_off(m, h, d, pos), t, lim, x);
  }
}

// GATED: the fallback pass of an MFMA prefill (returns at once unless the
// call's overflow mark is set; a grid of at most one workgroup per CU loops
// over the work items); otherwise one item per workgroup, with no loop or
// gate in the code.
template <int IODT, int KDT, int DMAX, bool GATED>
__global__ __launch_bounds__(256) void prologue_kernel(PrologueOp op) {
  __shared__ float sx[DMAX][kPT + 1];  // DMAX >= head_dim: the tile, sized to its class
  if constexpr (GATED) {  // fallback pass: runs only when this call's mark is set
    __shared__ unsigned s_go;
    if (threadIdx.x == 0) {
      const unsigned g = op.gate[1];
      s_go = op.gate[0] == g + 1u;
      if (blockIdx.x == 0 && blockIdx.y == 0) op.gate[2] = g + 1u;  // S for the fallback kernel
    }
    __syncthreads();
    if (!s_go) return;
  }
  __shared__ float scos[kTabHalf][kPT], ssin[kTabHalf][kPT];
  __shared__ float sred[8][kPT];
  __shared__ float sinv[kPT];
  __shared__ uint32_t smax[4];
  // Work item (tile, head group).
  const PrologueOp& op_k = op;
  auto run_item = [&](const int tile, const int hgrp) {
    // In the gated pass's item loop the parameters are read per item through
    // a kernel-argument pointer the compiler cannot see through (the
    // argument is the segment's only explicit one, at offset 0): otherwise
    // the loads are hoisted out of the loop and their values kept in SGPRs
    // across it, which spills them.
    typedef const __attribute__((address_space(4))) PrologueOp* kop_t;
    kop_t kp = nullptr;
    if constexpr (GATED) {
      kp = (kop_t)__builtin_amdgcn_kernarg_segment_ptr();
      asm volatile("" : "+s"(kp));
    }
    const PrologueOp& op = GATED ? *(const PrologueOp*)kp : op_k;
    const int tid = threadIdx.x;
    const int T = op.seq_len, D = op.head_dim;
    const int t0 = tile * kPT;
    const int n_vec = op.n_head + 2 * op.n_head_kv;
    // Work order idx -> head vector: with every head vector to do, the K and
    // V heads come first (the lowest workgroup ids, dispatched first: theirs
    // is the longer chain), then Q.
    const int nkv2 = 2 * op.n_head_kv;
    auto hv_of = [&](int idx) {
      if (op.hv_first != 0) return idx;
      return idx < nkv2 ? op.n_head + idx : idx - nkv2;
    };
    const int hv0 = op.hv_first + hgrp * op.hpg;  // work-order indices hv0 .. hv1 - 1
    const int hv1 = min(n_vec, hv0 + op.hpg);
    const int tc = tid & (kPT - 1), part = tid / kPT;  // 8 parts of 32 lanes
    const int t = t0 + tc;
    const int half = op.rope_dim / 2;
    // the (cos, sin) table when a Q or K head of the group is rotated
    const bool has_qk = op.hv_first != 0 ? hv0 < op.n_head + op.n_head_kv
                                         : (hv0 < op.n_head_kv || hv1 > nkv2);
    const bool tab = op.do_rope && half <= kTabHalf && has_qk;

    // Head vector hv -> (kind, head index, source); kind 0 q, 1 k, 2 v.
    auto decode_hv = [&](int hv, int& kind, int& h) {
      if (hv < op.n_head) {
        kind = 0;
        h = hv;
      } else if (hv < op.n_head + op.n_head_kv) {
        kind = 1;
        h = hv - op.n_head;
      } else {
        kind = 2;
        h = hv - op.n_head - op.n_head_kv;
      }
    };
    auto src_of = [&](int kind) { return kind == 0 ? op.q : (kind == 1 ? op.k : op.v); };
    // Loads head hv's [D, 32] tile into registers: thread -> (row, 8-token
    // chunk), 64 rows per pass, D <= 256 -> at most 4 passes.
    constexpr int kPass = DMAX / 64;
    const int c8 = (tid & 3) * 8;
    auto load_regs = [&](int hv, float (*x)[8]) {
      int kind, h;
      decode_hv(hv, kind, h);
      const void* src = src_of(kind);
      if (!src) return;
      const long long hbase = (long long)h * D * T;
  #pragma unroll
      for (int ps = 0; ps < kPass; ++ps) {
        const int r = (tid >> 2) + 64 * ps;
        if (r < D) load_row8_f32<IODT>(src, hbase + (long long)r * T + t0 + c8, t0 + c8, T, x[ps]);
      }
    };
    float xa[kPass][8], xb[kPass][8];
    if (hv0 < hv1) load_regs(hv_of(hv0), xa);  // in flight while the table is computed

    if (tab) {
      // The first head group's workgroup of each tile also publishes its slice
      // as tab_out[i][t] for the flash kernel's Q.
      const bool publish = op.rope_tab_out && hgrp == 0;
      const float pos = (float)(op.start_pos + t);
      for (int i = part; i < half; i += 8) {
        const float angle = pos * op.theta.t[i];
        float c, sn;
        rope_cs(angle, c, sn);
        scos[i][tc] = c;
        ssin[i][tc] = sn;
        if (publish && t < T) op.rope_tab_out[(long long)i * T + t] = make_float2(c, sn);
      }
    }


    for (int idx = hv0; idx < hv1; ++idx) {
      int kind, h;
      decode_hv(hv_of(idx), kind, h);
      const void* src = src_of(kind);
      // prefetch the next head's tile while this one is processed
      if (idx + 1 < hv1) load_regs(hv_of(idx + 1), xb);
      if (!src) {  // uniform across the workgroup
  #pragma unroll
        for (int ps = 0; ps < kPass; ++ps)
  #pragma unroll
          for (int e = 0; e < 8; ++e) xa[ps][e] = xb[ps][e];
        continue;
      }
      const float* nw = kind == 0 ? op.q_norm_w : (kind == 1 ? op.k_norm_w : nullptr);
      const bool rope = op.do_rope && kind < 2;
      const long long hbase = (long long)h * D * T;

      __syncthreads();  // previous head's readers of sx are done
  #pragma unroll
      for (int ps = 0; ps < kPass; ++ps) {
        const int r = (tid >> 2) + 64 * ps;
        if (r < D) {
  #pragma unroll
          for (int e = 0; e < 8; ++e) sx[r][c8 + e] = xa[ps][e];
        }
      }
  #pragma unroll
      for (int ps = 0; ps < kPass; ++ps)
  #pragma unroll
        for (int e = 0; e < 8; ++e) xa[ps][e] = xb[ps][e];
      __syncthreads();

      if (nw) {
        float ss = 0.f;
        for (int d = part; d < D; d += 8) ss += sx[d][tc] * sx[d][tc];
        sred[part][tc] = ss;
        __syncthreads();
        if (part == 0) {
          float tot = 0.f;
          for (int q = 0; q < 8; ++q) tot += sred[q][tc];
          sinv[tc] = 1.0f / sqrtf(tot / (float)D + op.eps);
        }
        __syncthreads();
        const float inv = sinv[tc];
        for (int d = part; d < D; d += 8) sx[d][tc] = sx[d][tc] * inv * nw[d];
        __syncthreads();
      }
      if (rope) {
        const float pos = (float)(op.start_pos + t);
        for (int i = part; i < half; i += 8) {
          int i0, i1;
          rope_pair_index(i, half, op.rope_style, i0, i1);
          float c, s;
          if (tab) {
            c = scos[i][tc];
            s = ssin[i][tc];
          } else {
            const float angle = pos * op.theta.t[i];
            rope_cs(angle, c, s);
          }
          const float v0 = sx[i0][tc], v1 = sx[i1][tc];
          sx[i0][tc] = v0 * c - v1 * s;
          sx[i1][tc] = v0 * s + v1 * c;
        }
        __syncthreads();
      }

      // row-wise outputs: fp32 write-back in place, KV-cache columns start_pos + t
      float* inplace = kind == 0 ? op.q_inplace : (kind == 1 ? op.k_inplace : op.v_f32);
      void* cache = kind == 1 ? op.k_cache : (kind == 2 ? op.v_cache : nullptr);
      if (inplace || cache) {
        for (int r = tid >> 2; r < D; r += 64) {
          float x[8];
  #pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = sx[r][c8 + e];
          if (inplace) store_row8<HL_F32>(inplace, hbase + (long long)r * T + t0 + c8, t0 + c8, T, x);
          if (cache)
            store_cache8<KDT>(cache, CacheMap{op.kv_layout, D, op.max_len, op.n_head_kv, op.block_table}, h, r,
                              op.start_pos + t0 + c8, t0 + c8, T, x);
        }
      }

      // Split images of the fp32 prefill (head dim 64 or 128): this tile is half
      // t0 / 32 % 2 of the 64-key image t0 / 64.  Scale: the largest
      // magnitude over the half (tokens past T are zeros); a half holding an
      // inf or NaN is flagged and not written.
      if (op.kv_img && kind >= 1 && (D == 64 || D == 128)) {
        const int hf = (t0 >> 5) & 1;
        const long long img_i = (long long)h * ((T + 63) >> 6) + (t0 >> 6);
        const int nper = D / 64;  // 16-byte pieces per thread: K (key, chunk), V (dim, 8 keys)
        // piece i: K key tid / 8, dims 8 ((tid % 8) + 8 i) + e; V dim tid / 4 + 64 i, keys c8 + e
        auto piece = [&](int i, int e) {
          return kind == 1 ? sx[8 * ((tid & 7) + 8 * i) + e][tid >> 3] : sx[(tid >> 2) + 64 * i][c8 + e];
        };
        uint32_t m = 0u;
        for (int i = 0; i < nper; ++i)
  #pragma unroll
          for (int e = 0; e < 8; ++e) m = max(m, __float_as_uint(piece(i, e)) & 0x7FFFFFFFu);
  #pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o, 64));
        if ((tid & 63) == 0) smax[tid >> 6] = m;
        __syncthreads();
        m = max(max(smax[0], smax[1]), max(smax[2], smax[3]));
        const bool bad = m >= kInfBits;
        const int sh = split_shift(m);
        if (tid == 0) {
          int* rec = op.kv_meta + img_i * kSplitRecInts;
          rec[(kind == 1 ? 0 : 2) + hf] = sh;
          rec[(kind == 1 ? 4 : 6) + hf] = bad ? 1 : 0;
        }
        if (!bad) {
          uint16_t* base = (uint16_t*)(op.kv_img + img_i * split_img_bytes(D));
          for (int i = 0; i < nper; ++i) {
            float x[8];
  #pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = __builtin_amdgcn_ldexpf(piece(i, e), sh);
            f16x8 h8, l8;
            split_f16x8(x, h8, l8);
            int pos;
            if (kind == 1) {
              const int key = 32 * hf + (tid >> 3), ch = (tid & 7) + 8 * i;
              pos = key * D + 8 * (ch ^ (key % (D / 8)));
            } else {
              const int r = (tid >> 2) + 64 * i, kc = 4 * hf + (c8 >> 3);
              pos = 2 * 64 * D + r * 64 + 8 * (kc ^ ((r >> 1) & 7));
            }
            *(f16x8*)(base + pos) = h8;
            *(f16x8*)(base + pos + 64 * D) = l8;
          }
        }
      }

      // MFMA operand layouts (fp16 bits); pad rows t >= T are written as zeros.
      // A value beyond fp16's range goes to the range record.
      float omax = 0.f;
      if (kind < 2) {
        uint16_t* dst = kind == 0 ? op.qt : op.kt;
        if (dst) {
          const float mul = kind == 0 ? op.qt_scale : 1.0f;
          const int chunks = D / 8;
          for (int idx = tid; idx < kPT * chunks; idx += 256) {
            const int tt = idx / chunks, ch = idx % chunks;
            const int tg = t0 + tt;
            if (tg >= op.t_pad) continue;
            u16x8 w;
  #pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float x = tg < T ? sx[8 * ch + e][tt] * mul : 0.f;
              omax = fmaxf(omax, fabsf(x));
              w[e] = f32_to_f16_bits(x);
            }
            *(u16x8*)(dst + ((long long)h * op.t_pad + tg) * D + 8 * ch) = w;
          }
        }
      } else if (op.vt) {
        for (int r = tid >> 2; r < D; r += 64) {
          if (t0 + c8 >= op.t_pad) continue;
          float x[8];
  #pragma unroll
          for (int e = 0; e < 8; ++e) {
            x[e] = (t0 + c8 + e < T) ? sx[r][c8 + e] : 0.f;
            omax = fmaxf(omax, fabsf(x[e]));
          }
          store_row8<HL_F16>(op.vt, ((long long)h * D + r) * op.t_pad + t0 + c8, t0 + c8, op.t_pad, x);
        }
      }
      if (omax >= kF16Inf && op.range_word) range_flag_set(op.range_word);
    }
  };
  if constexpr (GATED) {
    const int n_items = op.n_tiles * op.n_hgrps;
    for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
      run_item(item % op.n_tiles, item / op.n_tiles);
      __syncthreads();  // this item's LDS readers are done before the next item's fill
    }
  } else {
    run_item(blockIdx.x, blockIdx.y);
  }
}

// ---------------------------------------------------------------------------
// K/V prologue of an MFMA prefill whose Q the flash kernel builds itself.
// One workgroup per (32-token tile, kv head) handles that head's K and V with
// no fp32 staging: thread (r = tid / 4, c8 = 8 * (tid % 4)) holds rows r and
// r + 64 (D = 128) of 8 tokens.  Half-split RoPE over
// the whole head pairs rows r and r + D/2, which are in one thread;
// interleaved RoPE pairs rows 2i and 2i + 1, one lane-shuffle apart.  V goes
// from registers to the cache and to vt; only kt (token-major) is transposed,
// through a 32 x D fp16 LDS tile.  Formulas as the general prologue's:
// x * (1/sqrtf(ss/D + eps)) * w[d], (v0c - v1s, v0s + v1c), angle =
// float(start_pos + t) * theta[i].
// ---------------------------------------------------------------------------
// Column swizzle of the kt transposition tile: token rows t and t + 16 of
// the 272-byte-pitch tile start in the same bank, so the second half of the
// tokens stores its head dims XOR 16 (a whole 16-byte chunk pair, so the
// token-major readout still reads contiguous 16-byte chunks).
__device__ __forceinline__ int kt_swz(int tok) { return (tok & 16); }

// PT tokens per workgroup (32 or 64): a thread holds 8 tokens of rows
// r + RS * ps, RS = 256 / (PT / 8); 64-token tiles read and write 128-byte
// row segments instead of 64.
template <int IODT, int KDT, int D, int PT>
__global__ __launch_bounds__(256) void kv_prologue_kernel(PrologueOp op) {
  static_assert(D == 128, "half-split RoPE pairs rows r and r + 64 in-thread");
  constexpr int CPR = PT / 8;       // 8-token chunks per row
  constexpr int RS = 256 / CPR;     // rows per pass
  constexpr int NP = D / RS;        // row passes: rows r + RS * ps
  __shared__ __attribute__((aligned(16))) uint16_t skt[PT][D + 8];  // kt tile (fp16 bits), padded rows
  __shared__ float sred[4][PT];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = op.seq_len;
  const int t0 = blockIdx.x * PT;
  const int h = blockIdx.y;
  const int r = tid / CPR, c8 = (tid % CPR) * 8;
  const int t = t0 + c8;  // this thread's first token
  const long long hbase = (long long)h * D * T;

  float k[NP][8], v[NP][8];
#pragma unroll
  for (int ps = 0; ps < NP; ++ps) {
    load_row8_f32<IODT>(op.k, hbase + (long long)(r + RS * ps) * T + t, t, T, k[ps]);
    load_row8_f32<IODT>(op.v, hbase + (long long)(r + RS * ps) * T + t, t, T, v[ps]);
  }

  // V: cache column block and vt, straight from registers.  omax: the
  // largest operand magnitude this thread converts (range record).
  float omax = 0.f;
#pragma unroll
  for (int ps = 0; ps < NP; ++ps) {
    const int row = r + RS * ps;
    if (op.v_cache)
      store_cache8<KDT>(op.v_cache, CacheMap{op.kv_layout, D, op.max_len, op.n_head_kv, op.block_table}, h, row,
                        op.start_pos + t, t, T, v[ps]);
    if (t < op.t_pad) {
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[e] = t + e < T ? v[ps][e] : 0.f;
        omax = fmaxf(omax, fabsf(x[e]));
      }
      store_row8<HL_F16>(op.vt, ((long long)h * D + row) * op.t_pad + t, t, op.t_pad, x);
    }
  }

  // K: RMSNorm over the head dimension per token.
  if (op.k_norm_w) {
    float ss[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float a = 0.f;
#pragma unroll
      for (int ps = 0; ps < NP; ++ps) a += k[ps][e] * k[ps][e];
      // lanes with the same c8 (tid % CPR) hold the other rows of this wave
#pragma unroll
      for (int m = CPR; m < 64; m <<= 1) a += __shfl_xor(a, m, 64);
      ss[e] = a;
    }
    if (lane < CPR) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sred[wave][c8 + e] = ss[e];
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float tot = sred[0][c8 + e] + sred[1][c8 + e] + sred[2][c8 + e] + sred[3][c8 + e];
      const float inv = 1.0f / sqrtf(tot / (float)D + op.eps);
#pragma unroll
      for (int ps = 0; ps < NP; ++ps) k[ps][e] = k[ps][e] * inv * op.k_norm_w[r + RS * ps];
    }
  }

  // K: RoPE at positions start_pos + t.  The kv head 0 workgroup of each tile
  // publishes the (cos, sin) of its tokens for the flash kernel's Q.
  if (op.do_rope) {
    const bool publish = op.rope_tab_out && h == 0;
    const int half = op.rope_dim / 2;
    if (op.rope_style == HL_ROPE_HALF_SPLIT) {  // rope_dim == D: pair (row, row + 64) = passes (ps, ps + NP/2)
#pragma unroll
      for (int ps = 0; ps < NP / 2; ++ps) {
        const int i = r + RS * ps;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float angle = (float)(op.start_pos + t + e) * op.theta.t[i];
          float c, sn;
          rope_cs(angle, c, sn);
          const float v0 = k[ps][e], v1 = k[ps + NP / 2][e];
          k[ps][e] = v0 * c - v1 * sn;
          k[ps + NP / 2][e] = v0 * sn + v1 * c;
          if (publish && t + e < T) op.rope_tab_out[(long long)i * T + t + e] = make_float2(c, sn);
        }
      }
    } else {  // interleaved: rows 2i and 2i + 1 are lanes CPR apart
      const bool even = (r & 1) == 0;
#pragma unroll
      for (int ps = 0; ps < NP; ++ps) {
        const int row = r + RS * ps;
        const int i = row >> 1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float other = __shfl_xor(k[ps][e], CPR, 64);
          if (row < op.rope_dim) {
            const float angle = (float)(op.start_pos + t + e) * op.theta.t[i];
            float c, sn;
            rope_cs(angle, c, sn);
            const float v0 = even ? k[ps][e] : other, v1 = even ? other : k[ps][e];
            k[ps][e] = even ? v0 * c - v1 * sn : v0 * sn + v1 * c;
            if (publish && even && t + e < T) op.rope_tab_out[(long long)i * T + t + e] = make_float2(c, sn);
          }
        }
      }
    }
  }

  // K: cache column block, and kt through LDS (token-major fp16).
#pragma unroll
  for (int ps = 0; ps < NP; ++ps) {
    const int row = r + RS * ps;
    if (op.k_cache)
      store_cache8<KDT>(op.k_cache, CacheMap{op.kv_layout, D, op.max_len, op.n_head_kv, op.block_table}, h, row,
                        op.start_pos + t, t, T, k[ps]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = t + e < T ? k[ps][e] : 0.f;
      omax = fmaxf(omax, fabsf(x));
      skt[c8 + e][row ^ kt_swz(c8 + e)] = f32_to_f16_bits(x);
    }
  }
  if (omax >= kF16Inf && op.range_word) range_flag_set(op.range_word);
  __syncthreads();
  constexpr int CH = D / 8;  // 16-byte chunks per token row
  for (int idx = tid; idx < PT * CH; idx += 256) {
    const int tt = idx / CH, ch = idx % CH;
    const int tg = t0 + tt;
    if (tg < op.t_pad) *(u16x8*)(op.kt + ((long long)h * op.t_pad + tg) * D + 8 * ch) = *(const u16x8*)&skt[tt][(8 * ch) ^ kt_swz(tt)];
  }
}

// True when kv_prologue_kernel covers the op: K/V only, MFMA layouts, and a
// RoPE whose pairs it holds in-thread or one shuffle apart.
static bool kv_prologue_fits(const PrologueOp& op) {
  if (op.q || op.q_inplace || op.k_inplace || !op.kt || !op.vt) return false;
  if (op.hv_first != op.n_head) return false;
  if (op.head_dim != 128) return false;
  if (op.do_rope && op.rope_style == HL_ROPE_HALF_SPLIT && op.rope_dim != op.head_dim) return false;
  return true;
}

hipError_t prologue_launch(const PrologueOp& op, hipStream_t stream) {
  const int cols = op.t_pad > op.seq_len ? op.t_pad : op.seq_len;
  if (kv_prologue_fits(op)) {
    constexpr int PT = 32;  // 64-token tiles (128-byte row segments) measured 0.8% slower at c4
    dim3 grid((cols + PT - 1) / PT, op.n_head_kv);
#define HL_KVP(IO, KD) hipLaunchKernelGGL((kv_prologue_kernel<IO, KD, 128, PT>), grid, dim3(256), 0, stream, op)
    const int kd = op.k_cache ? op.kv_dtype : HL_BF16;
    if (op.io_dtype == HL_F16) {
      if (kd == HL_F32) HL_KVP(HL_F16, HL_F32); else if (kd == HL_F16) HL_KVP(HL_F16, HL_F16);
      else if (kd == HL_FP8) HL_KVP(HL_F16, HL_FP8); else HL_KVP(HL_F16, HL_BF16);
    } else {
      if (kd == HL_F32) HL_KVP(HL_BF16, HL_F32); else if (kd == HL_F16) HL_KVP(HL_BF16, HL_F16);
      else if (kd == HL_FP8) HL_KVP(HL_BF16, HL_FP8); else HL_KVP(HL_BF16, HL_BF16);
    }
#undef HL_KVP
    return hipGetLastError();
  }
  const int n_vec = op.n_head + 2 * op.n_head_kv - op.hv_first;
  const int tiles = (cols + kPT - 1) / kPT;
  // Head vectors per workgroup: enough workgroups (~2048) to keep every CU
  // busy through the load latency of a tile, and up to kHPG so that small
  // prefills share one cos/sin table fill across heads.
  PrologueOp o2 = op;
  o2.hpg = kHPG;
  while (!op.gate && o2.hpg > 1 && (long long)tiles * ((n_vec + o2.hpg - 1) / o2.hpg) < 2048) o2.hpg >>= 1;
  o2.n_tiles = tiles;
  o2.n_hgrps = (n_vec + o2.hpg - 1) / o2.hpg;
  // A gated fallback pass usually exits at once: one workgroup per CU at
  // most (one round of gate reads), looping over the items when it runs.
  dim3 grid = op.gate ? dim3(std::min(tiles * o2.n_hgrps, cu_count())) : dim3(tiles, o2.n_hgrps);
#define HL_PRO_G(IO, KD, G)                                                                     \
  if (op.head_dim <= 128) hipLaunchKernelGGL((prologue_kernel<IO, KD, 128, G>), grid, dim3(256), 0, stream, o2); \
  else hipLaunchKernelGGL((prologue_kernel<IO, KD, HL_MAX_HEAD_DIM, G>), grid, dim3(256), 0, stream, o2)
#define HL_PRO(IO, KD)             \
  if (op.gate) {                   \
    HL_PRO_G(IO, KD, true);        \
  } else {                         \
    HL_PRO_G(IO, KD, false);       \
  }
#define HL_PRO_IO(IO)                      \
  switch (op.kv_dtype) {                   \
    case HL_F32: HL_PRO(IO, HL_F32); break; \
    case HL_F16: HL_PRO(IO, HL_F16); break; \
    case HL_FP8: HL_PRO(IO, HL_FP8); break; \
    default: HL_PRO(IO, HL_BF16); break;    \
  }
  switch (op.io_dtype) {
    case HL_F32: HL_PRO_IO(HL_F32); break;
    case HL_F16: HL_PRO_IO(HL_F16); break;
    default: HL_PRO_IO(HL_BF16); break;
  }
#undef HL_PRO_IO
#undef HL_PRO
#undef HL_PRO_G
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// storeKV / storeKVPair: [rows, src_cols] fp32 -> cache columns start_pos..
// ---------------------------------------------------------------------------
template <int KDT>
__global__ __launch_bounds__(256) void store_cols_kernel(void* cache, const float* src, void* cache2,
                                                         const float* src2, int rows, int src_cols,
                                                         int cache_cols, int start_pos) {
  const long long total = (long long)rows * src_cols;
  long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  const bool second = idx >= total;
  if (second) {
    if (!src2) return;
    idx -= total;
    if (idx >= total) return;
  }
  const int r = (int)(idx / src_cols), c = (int)(idx % src_cols);
  const float v = (second ? src2 : src)[idx];
  store_elem<KDT>(second ? cache2 : cache, (long long)r * cache_cols + start_pos + c, v);
}

hipError_t store_cols_launch(void* cache, const float* src, void* cache2, const float* src2,
                             int rows, int src_cols, int cache_cols, int start_pos, int kv_dtype,
                             hipStream_t stream) {
  const long long total = (long long)rows * src_cols * (src2 ? 2 : 1);
  dim3 grid((unsigned)((total + 255) / 256));
  switch (kv_dtype) {
    case HL_F32:
      hipLaunchKernelGGL(store_cols_kernel<HL_F32>, grid, dim3(256), 0, stream, cache, src, cache2,
                         src2, rows, src_cols, cache_cols, start_pos);
      break;
    case HL_F16:
      hipLaunchKernelGGL(store_cols_kernel<HL_F16>, grid, dim3(256), 0, stream, cache, src, cache2,
                         src2, rows, src_cols, cache_cols, start_pos);
      break;
    default:
      hipLaunchKernelGGL(store_cols_kernel<HL_BF16>, grid, dim3(256), 0, stream, cache, src, cache2,
                         src2, rows, src_cols, cache_cols, start_pos);
      break;
  }
  return hipGetLastError();
}

template <int KDT>
__global__ __launch_bounds__(256) void cache_to_f32_kernel(float* dst, const void* cache, int rows,
                                                           int max_len, int col0, int ncols) {
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long long)rows * ncols) return;
  const int r = (int)(idx / ncols), c = (int)(idx % ncols);
  dst[idx] = load_elem<KDT>(cache, (long long)r * max_len + col0 + c);
}

hipError_t cache_to_f32_launch(float* dst, const void* cache, int kv_dtype, int rows, int max_len,
                               int col0, int ncols, hipStream_t stream) {
  dim3 grid((unsigned)(((long long)rows * ncols + 255) / 256));
  switch (kv_dtype) {
    case HL_F32:
      hipLaunchKernelGGL(cache_to_f32_kernel<HL_F32>, grid, dim3(256), 0, stream, dst, cache, rows,
                         max_len, col0, ncols);
      break;
    case HL_F16:
      hipLaunchKernelGGL(cache_to_f32_kernel<HL_F16>, grid, dim3(256), 0, stream, dst, cache, rows,
                         max_len, col0, ncols);
      break;
    case HL_FP8:
      hipLaunchKernelGGL(cache_to_f32_kernel<HL_FP8>, grid, dim3(256), 0, stream, dst, cache, rows,
                         max_len, col0, ncols);
      break;
    default:
      hipLaunchKernelGGL(cache_to_f32_kernel<HL_BF16>, grid, dim3(256), 0, stream, dst, cache, rows,
                         max_len, col0, ncols);
      break;
  }
  return hipGetLastError();
}

}  // namespace hl
