// One greedy decode step of a dense decoder, host side above the C ABI: the
// forwardDecodeToken layer loop of the reference for layers of kind
// lkAttentionFfn (backends/naive.nim:4592-4760 and 5520-5545), issuing the
// library's own entry points in the reference's order on one stream, plus
// the two elementwise kernels that loop needs (gpuSiluMul, gpuAdd).
//
// Everything stays on the device between steps: the token is read from and
// the next token written to device memory, so consecutive steps chain
// without a host round trip.
#include <cmath>

#include "common.h"
#include "launch.h"

namespace hl {
namespace {

// silu(g) * u with silu(g) = g / (1 + e^-g), as g * (1 / (1 + expf(-g))) * u
// (naive.nim:2179-2187).
__global__ __launch_bounds__(256) void silu_mul_kernel(float* __restrict__ dst, const float* gate,
                                                       const float* up, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    const float g = gate[i];
    dst[i] = g * (1.0f / (1.0f + expf(-g))) * up[i];
  }
}

__global__ __launch_bounds__(256) void add_kernel(float* dst, const float* a, const float* b, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = a[i] + b[i];
}

}  // namespace
}  // namespace hl

using namespace hl;

extern "C" {

int hl_gpu_silu_mul(float* dst, const float* gate, const float* up, int n, void* stream) {
  if (!dst || !gate || !up) return set_error(HL_EINVAL, "silu_mul: null pointer");
  if (n <= 0) return set_error(HL_EINVAL, "silu_mul: bad size %d", n);
  hipLaunchKernelGGL(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, dst,
                     gate, up, n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? HL_OK : set_error(HL_EHIP, "silu_mul launch: %s", hipGetErrorString(e));
}

int hl_gpu_add(float* dst, const float* a, const float* b, int n, void* stream) {
  if (!dst || !a || !b) return set_error(HL_EINVAL, "add: null pointer");
  if (n <= 0) return set_error(HL_EINVAL, "add: bad size %d", n);
  hipLaunchKernelGGL(add_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, dst, a, b, n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? HL_OK : set_error(HL_EHIP, "add launch: %s", hipGetErrorString(e));
}

// Shape / type checks of the fused quantized GEMVs (as hl_gpu_linear_col_quant).
static int check_quant_pair(const void* d0, const void* d1, const float* x, const void* wa,
                            const void* wb, int w_cols, int w_rows, int ta, int tb, const char* who) {
  if (!d0 || !d1 || !x || !wa || !wb) return set_error(HL_EINVAL, "%s: null pointer", who);
  if (w_cols <= 0 || w_rows <= 0)
    return set_error(HL_EINVAL, "%s: bad shape (w_cols=%d, w_rows=%d)", who, w_cols, w_rows);
  for (int t : {ta, tb}) {
    const int qk = quant_block_elems(t);
    if (qk == 0) return set_error(HL_EUNSUPPORTED, "unsupported quant type for GPU GEMV: %d", t);
    if (t != HL_GGML_F16 && w_cols % qk)
      return set_error(HL_EINVAL, "%s: row size must be multiple of %d", who, qk);
  }
  return HL_OK;
}

// gpuFusedGateUpSiluQ4K / Q3K (naive.nim:1905-1920, 1693-1708), any one GGUF
// type: dst = silu(W_gate x) * (W_up x) in one launch.  Needs x 16-byte
// aligned and the weights aligned as their blocks (the direct kernel);
// HL_EINVAL otherwise (the reference's fused kernels have their own limits:
// wave32 builds only).
int hl_gpu_fused_gate_up_silu_quant(float* dst, const float* x, const void* gate_q, const void* up_q,
                                    int w_cols, int w_rows, int quant_type, void* stream) {
  const int rc = check_quant_pair(dst, dst, x, gate_q, up_q, w_cols, w_rows, quant_type, quant_type,
                                  "fused_gate_up_silu");
  if (rc != HL_OK) return rc;
  if (!linear_quant_pair_launch(1, dst, nullptr, x, gate_q, up_q, w_cols, w_rows, quant_type,
                                (hipStream_t)stream))
    return set_error(HL_EINVAL, "fused_gate_up_silu: x must be 16-byte aligned and the weights "
                                "aligned to their block layout");
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? HL_OK : set_error(HL_EHIP, "fused_gate_up_silu launch: %s", hipGetErrorString(e));
}

// gpuFusedKVLinearQ4K / Q2KQ3K (naive.nim:1799-1814, 853-868), any GGUF
// types: k_dst = W_k x, v_dst = W_v x.  One launch when both have one type
// and the direct kernel takes the pointers, otherwise two.
int hl_gpu_fused_kv_linear_quant(float* k_dst, float* v_dst, const float* x, const void* k_q,
                                 const void* v_q, int w_cols, int w_rows, int k_type, int v_type,
                                 void* stream) {
  const int rc = check_quant_pair(k_dst, v_dst, x, k_q, v_q, w_cols, w_rows, k_type, v_type,
                                  "fused_kv_linear");
  if (rc != HL_OK) return rc;
  if (k_type == v_type && linear_quant_pair_launch(2, k_dst, v_dst, x, k_q, v_q, w_cols, w_rows,
                                                    k_type, (hipStream_t)stream)) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? HL_OK : set_error(HL_EHIP, "fused_kv_linear launch: %s", hipGetErrorString(e));
  }
  const int r1 = hl_gpu_linear_col_quant(k_dst, x, k_q, w_cols, w_rows, k_type, stream);
  return r1 != HL_OK ? r1 : hl_gpu_linear_col_quant(v_dst, x, v_q, w_cols, w_rows, v_type, stream);
}

// The reference's names (same argument order).
int hl_gpu_fused_gate_up_silu_q4k(float* dst, const float* x, const void* gate_q, const void* up_q,
                                  int w_cols, int w_rows, void* stream) {
  return hl_gpu_fused_gate_up_silu_quant(dst, x, gate_q, up_q, w_cols, w_rows, HL_GGML_Q4_K, stream);
}
int hl_gpu_fused_gate_up_silu_q3k(float* dst, const float* x, const void* gate_q, const void* up_q,
                                  int w_cols, int w_rows, void* stream) {
  return hl_gpu_fused_gate_up_silu_quant(dst, x, gate_q, up_q, w_cols, w_rows, HL_GGML_Q3_K, stream);
}
int hl_gpu_fused_kv_linear_q4k(float* k_dst, float* v_dst, const float* x, const void* k_q,
                               const void* v_q, int w_cols, int w_rows, void* stream) {
  return hl_gpu_fused_kv_linear_quant(k_dst, v_dst, x, k_q, v_q, w_cols, w_rows, HL_GGML_Q4_K,
                                      HL_GGML_Q4_K, stream);
}
int hl_gpu_fused_kv_linear_q2k_q3k(float* k_dst, float* v_dst, const float* x, const void* k_q,
                                   const void* v_q, int w_cols, int w_rows, void* stream) {
  return hl_gpu_fused_kv_linear_quant(k_dst, v_dst, x, k_q, v_q, w_cols, w_rows, HL_GGML_Q2_K,
                                      HL_GGML_Q3_K, stream);
}

// y[rows] = W[rows, cols] . x: gpuLinearCol (fp32) or gpuLinearColQuant.
static int linear(float* y, const float* x, const void* w, int type, int cols, int rows, void* stream) {
  return type == 0 ? hl_gpu_linear_col(y, x, (const float*)w, cols, rows, 1, stream)
                   : hl_gpu_linear_col_quant(y, x, w, cols, rows, type, stream);
}

#define HL_TRY(call)              \
  do {                            \
    const int rc_ = (call);       \
    if (rc_ != HL_OK) return rc_; \
  } while (0)

int hl_forward_decode_token(const hl_model_desc* m, const hl_decode_scratch* s,
                            const int32_t* token_dev, int pos, float* logits,
                            int32_t* next_token_dev, void* stream) {
  if (!m || !s || !token_dev || !logits || !next_token_dev || !m->layers || !m->tok_emb ||
      !m->output_norm || !m->output || !s->x || !s->x_norm || !s->tmp0 || !s->tmp1 || !s->tmp2)
    return set_error(HL_EINVAL, "forward_decode_token: null pointer");
  if (m->n_layer <= 0 || m->n_emb <= 0 || m->n_head <= 0 || m->n_head_kv <= 0 || m->head_dim <= 0 ||
      m->n_ff <= 0 || m->n_vocab <= 0 || m->max_len <= 0)
    return set_error(HL_EINVAL, "forward_decode_token: bad model shape");
  if (pos < 0 || pos >= m->max_len)
    return set_error(HL_ECAPACITY, "forward_decode_token: position %d outside the cache (%d)", pos,
                   m->max_len);
  const int E = m->n_emb, D = m->head_dim, qdim = m->n_head * D, kvdim = m->n_head_kv * D;
  const float eps = m->rms_eps;
  HL_TRY(hl_set_rope_theta(m->rope_dim, m->rope_base));
  HL_TRY(hl_gpu_embedding(s->x, m->tok_emb, token_dev, E, 1, m->n_vocab, stream));
  HL_TRY(hl_gpu_rmsnorm_cols(s->x_norm, s->x, m->layers[0].attn_norm, E, 1, eps, stream));
  for (int l = 0; l < m->n_layer; ++l) {
    const hl_layer_desc& L = m->layers[l];
    HL_TRY(linear(s->tmp0, s->x_norm, L.wq, L.wq_type, E, qdim, stream));
    // K and V in one launch when they share a GGUF type (the reference's
    // fused K/V GEMVs), else apart.
    if (!(L.wk_type != 0 && L.wk_type == L.wv_type &&
          linear_quant_pair_launch(2, s->tmp1, s->tmp2, s->x_norm, L.wk, L.wv, E, kvdim, L.wk_type,
                                   (hipStream_t)stream))) {
      HL_TRY(linear(s->tmp1, s->x_norm, L.wk, L.wk_type, E, kvdim, stream));
      HL_TRY(linear(s->tmp2, s->x_norm, L.wv, L.wv_type, E, kvdim, stream));
    }
    if (L.q_norm) HL_TRY(hl_gpu_qk_norm(s->tmp0, L.q_norm, m->n_head, D, eps, stream));
    if (L.k_norm) HL_TRY(hl_gpu_qk_norm(s->tmp1, L.k_norm, m->n_head_kv, D, eps, stream));
    HL_TRY(hl_gpu_rope_qk_decode(s->tmp0, s->tmp1, m->n_head, m->n_head_kv, D, m->rope_dim,
                                 m->rope_base, pos, stream));
    HL_TRY(hl_gpu_store_kv_pair(L.k_cache, s->tmp1, L.v_cache, s->tmp2, kvdim, 1, m->max_len, pos,
                                stream));
    HL_TRY(hl_gpu_attention_decode(s->x_norm, s->tmp0, L.k_cache, L.v_cache, m->n_head, m->n_head_kv,
                                   D, pos + 1, m->max_len, stream));
    HL_TRY(linear(s->tmp0, s->x_norm, L.wo, L.wo_type, qdim, E, stream));
    HL_TRY(hl_gpu_residual_rmsnorm(s->x_norm, s->x, s->tmp0, L.ffn_norm, E, eps, stream));
    // gate, up and SiLU * up in one launch when gate and up share a GGUF
    // type (the reference's fused gate/up/SiLU GEMVs), else apart.
    if (!(L.w_gate_type != 0 && L.w_gate_type == L.w_up_type &&
          linear_quant_pair_launch(1, s->tmp2, nullptr, s->x_norm, L.w_gate, L.w_up, E, m->n_ff,
                                   L.w_gate_type, (hipStream_t)stream))) {
      HL_TRY(linear(s->tmp0, s->x_norm, L.w_gate, L.w_gate_type, E, m->n_ff, stream));
      HL_TRY(linear(s->tmp1, s->x_norm, L.w_up, L.w_up_type, E, m->n_ff, stream));
      HL_TRY(hl_gpu_silu_mul(s->tmp2, s->tmp0, s->tmp1, m->n_ff, stream));
    }
    HL_TRY(linear(s->tmp0, s->tmp2, L.w_down, L.w_down_type, m->n_ff, E, stream));
    if (l + 1 < m->n_layer)
      HL_TRY(hl_gpu_residual_rmsnorm(s->x_norm, s->x, s->tmp0, m->layers[l + 1].attn_norm, E, eps, stream));
    else
      HL_TRY(hl_gpu_add(s->x, s->x, s->tmp0, E, stream));
  }
  HL_TRY(hl_gpu_rmsnorm_cols(s->x_norm, s->x, m->output_norm, E, 1, eps, stream));
  HL_TRY(linear(logits, s->x_norm, m->output, m->output_type, E, m->n_vocab, stream));
  return hl_argmax_async(logits, m->n_vocab, next_token_dev, stream);
}

}  // extern "C"
