// The two ends of a decode step around the layers: the token embedding
// lookup in front (gpuEmbedding, backends/naive.nim:2975-3001) and the
// greedy argmax over the logits behind the output projection (gpuArgmax,
// naive.nim:1922-2127, called at naive.nim:5544).  Both are HBM- or
// latency-bound byte work.
//
// argmax_kernel: one launch.  Each workgroup reduces its share of the logits
// to one 64-bit key, the last workgroup to arrive folds the keys and writes
// the index.  The key reproduces the reference's result exactly, including
// the tie-break its reduction tree implies and the values it never selects
// (see argmax_key).
//
// embedding_kernel: out[e, t] = W[tok[t], e] with out column-major
// [nEmb, T]: rows of W are read along e, written along t, through an LDS
// tile of 64 tokens x 64 dims.
#include "common.h"
#include "launch.h"

namespace hl {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// The reference (naive.nim:1922-2103) scans with 256 blocks x 256 threads:
// thread (b, t) keeps the first strictly greater value among elements
// i = 65536 r + 256 b + t (r = 0, 1, ...), starting from -3.4e38.  Its block
// reduction (steps 128, 64, then shuffles 32 .. 1) and the second pass over
// the 256 block results replace a value only when the other is strictly
// greater, so on a tie the lower position of each merge wins.  The last
// merge (position bit 0) decides first: among equal maxima the winner is
// the one with the smallest (bitrev8(b), bitrev8(t), r).  Values that are
// not greater than -3.4e38 (NaN, -inf, anything <= -3.4e38) are never
// taken, and if no element is taken the result is -1.
//
// The key orders elements the same way: high word = value as an
// order-preserving integer (-0 folded onto +0: the reference's > treats them
// as equal), low word = 2^31 - 1 - (bitrev8(b) << 23 | bitrev8(t) << 15 | r);
// untaken elements get key 0.  Valid for n < 2^31.
__device__ __forceinline__ unsigned int bitrev8(unsigned int v) {
  return __builtin_bitreverse32(v) >> 24;
}

__device__ __forceinline__ unsigned long long argmax_key(float v, int i) {
  if (!(v > -3.4e38f)) return 0ull;
  v += 0.0f;  // -0 -> +0
  const unsigned int u = __float_as_uint(v);
  const unsigned int hi = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  const unsigned int ui = (unsigned int)i;
  const unsigned int tb = bitrev8((ui >> 8) & 255u) << 23 | bitrev8(ui & 255u) << 15 | (ui >> 16);
  return ((unsigned long long)hi << 32) | (0x7FFFFFFFu - tb);
}

__device__ __forceinline__ int key_index(unsigned long long k) {
  if (k == 0ull) return -1;
  const unsigned int tb = 0x7FFFFFFFu - (unsigned int)(k & 0xFFFFFFFFull);
  return (int)((tb & 0x7FFFu) << 16 | bitrev8(tb >> 23) << 8 | bitrev8((tb >> 15) & 255u));
}

__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}

__device__ __forceinline__ unsigned long long wave_max64(unsigned long long k) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) k = umax64(k, __shfl_xor(k, o, 64));
  return k;
}

// Workgroup max of one key per thread (256 threads).
__device__ __forceinline__ unsigned long long block_max64(unsigned long long k) {
  __shared__ unsigned long long part[4];
  k = wave_max64(k);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = k;
  __syncthreads();
  return umax64(umax64(part[0], part[1]), umax64(part[2], part[3]));
}

// Scratch layout (library-owned, per device): [0] arrival counter (u32,
// zero between calls), [8..] one key per workgroup.
template <bool VEC>
__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ x, int n,
                                                     unsigned int* scratch, int* result) {
  unsigned long long* keys = (unsigned long long*)(scratch + 2);
  const int G = gridDim.x;
  unsigned long long best = 0ull;
  if (VEC) {
    const int n4 = n >> 2;
    const f32x4* x4 = (const f32x4*)x;
    for (int j = blockIdx.x * 256 + threadIdx.x; j < n4; j += G * 256) {
      const f32x4 v = __builtin_nontemporal_load(&x4[j]);
      best = umax64(best, argmax_key(v.x, 4 * j));
      best = umax64(best, argmax_key(v.y, 4 * j + 1));
      best = umax64(best, argmax_key(v.z, 4 * j + 2));
      best = umax64(best, argmax_key(v.w, 4 * j + 3));
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
      const int i = (n & ~3) + threadIdx.x;
      best = umax64(best, argmax_key(x[i], i));
    }
  } else {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += G * 256)
      best = umax64(best, argmax_key(x[i], i));
  }
  best = block_max64(best);
  if (G == 1) {
    if (threadIdx.x == 0) *result = key_index(best);
    return;
  }
  // Partials are exchanged with relaxed agent-scope atomics (coherent across
  // the XCDs' L2s); each writer's store completes before the barrier that
  // precedes its arrival RMW, and the last workgroup reads after the RMW.
  __shared__ int s_last;
  if (threadIdx.x == 0) __hip_atomic_store(&keys[blockIdx.x], best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // s_waitcnt vmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned int old = __hip_atomic_fetch_add(scratch, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = old == (unsigned int)(G - 1);
  }
  __syncthreads();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  if (!s_last) return;
  unsigned long long k = 0ull;
  for (int b = threadIdx.x; b < G; b += 256)
    k = umax64(k, __hip_atomic_load(&keys[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  k = block_max64(k);
  if (threadIdx.x == 0) {
    *result = key_index(k);
    __hip_atomic_store(scratch, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// 64 tokens x 64 dims per workgroup; token ids outside [0, n_vocab) give a
// NaN column (the reference reads out of bounds there).
__global__ __launch_bounds__(256) void embedding_kernel(const float* __restrict__ w,
                                                        const int* __restrict__ tok,
                                                        float* __restrict__ out, int n_emb,
                                                        int n_tok, int n_vocab) {
  __shared__ float tile[64][65];
  const int e0 = blockIdx.x * 64, t0 = blockIdx.y * 64;
  const int c = threadIdx.x & 63, r0 = threadIdx.x >> 6;
#pragma unroll 4
  for (int r = r0; r < 64; r += 4) {
    const int t = t0 + r, e = e0 + c;
    float v = 0.f;
    if (t < n_tok && e < n_emb) {
      const int id = tok[t];
      v = (id >= 0 && id < n_vocab) ? w[(size_t)id * n_emb + e] : __builtin_nanf("");
    }
    tile[r][c] = v;
  }
  __syncthreads();
#pragma unroll 4
  for (int r = r0; r < 64; r += 4) {
    const int e = e0 + r, t = t0 + c;
    if (e < n_emb && t < n_tok) out[(size_t)e * n_tok + t] = tile[c][r];
  }
}

}  // namespace

int argmax_grid(int n) {
  // ~8 KB of logits per workgroup, at most 256 workgroups (2 KB keys).
  const int g = (n + 2047) / 2048;
  return g < 1 ? 1 : (g > kArgmaxMaxGroups ? kArgmaxMaxGroups : g);
}

hipError_t argmax_launch(const float* x, int n, unsigned int* scratch, int* result,
                         hipStream_t stream) {
  const int G = argmax_grid(n);
  const bool vec = ((uintptr_t)x & 15) == 0;
  if (vec) hipLaunchKernelGGL(argmax_kernel<true>, dim3(G), dim3(256), 0, stream, x, n, scratch, result);
  else hipLaunchKernelGGL(argmax_kernel<false>, dim3(G), dim3(256), 0, stream, x, n, scratch, result);
  return hipGetLastError();
}

hipError_t embedding_launch(float* out, const float* w, const int* tok, int n_emb, int n_tok,
                            int n_vocab, hipStream_t stream) {
  const dim3 grid((n_emb + 63) / 64, (n_tok + 63) / 64);
  hipLaunchKernelGGL(embedding_kernel, grid, dim3(256), 0, stream, w, tok, out, n_emb, n_tok, n_vocab);
  return hipGetLastError();
}

}  // namespace hl
