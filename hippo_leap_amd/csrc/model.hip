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
#include <cstring>
#include <mutex>

#include "common.h"
#include "launch.h"

namespace hl {
namespace {

// silu(g) * u with silu(g) = g / (1 + e^-g), as g * (1 / (1 + expf(-g))) * u
// (naive.nim:2179-2187).
// dst may alias gate or up (the reference's MoE path calls it in place).
__global__ __launch_bounds__(256) void silu_mul_kernel(float* dst, const float* gate, const float* up, int n) {
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

// The fused two-matrix GEMV reads F16 rows in 8-weight groups; other row
// lengths go through two single GEMVs.
static bool pair_fusable(int type, int w_cols) { return type != HL_GGML_F16 || w_cols % 8 == 0; }

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
  if (!pair_fusable(quant_type, w_cols))
    return set_error(HL_EINVAL, "fused_gate_up_silu: F16 rows must hold a multiple of 8 weights (got %d)", w_cols);
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
  if (k_type == v_type && pair_fusable(k_type, w_cols) &&
      linear_quant_pair_launch(2, k_dst, v_dst, x, k_q, v_q, w_cols, w_rows, k_type, (hipStream_t)stream)) {
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

// ---------------------------------------------------------------------------
// Up-front checks: a forward call validates every shape, pointer and
// per-layer call before its first launch, so a refused call has no side
// effects (no half-written caches or scratch).
// ---------------------------------------------------------------------------
static int rope_dim_of(const hl_model_desc* m) { return m->rope_dim > 0 ? m->rope_dim : m->head_dim; }

static int check_weight(const void* w, int type, int cols, const char* what, int layer, bool fp32_only) {
  if (!w) return set_error(HL_EINVAL, "model: layer %d %s is null", layer, what);
  if (type == 0) return HL_OK;
  if (fp32_only)
    return set_error(HL_EUNSUPPORTED, "prefill: layer %d %s is GGUF type %d; prefill takes fp32 weights "
                                      "(as the reference's forwardPrefill)", layer, what, type);
  const int qk = quant_block_elems(type);
  if (qk == 0) return set_error(HL_EUNSUPPORTED, "unsupported quant type for GPU GEMV: %d", type);
  if (type != HL_GGML_F16 && cols % qk)
    return set_error(HL_EINVAL, "model: layer %d %s: row size must be multiple of %d", layer, what, qk);
  return HL_OK;
}

static int check_model(const hl_model_desc* m, bool fp32_only) {
  if (!m || !m->layers || !m->tok_emb || !m->output_norm || !m->output)
    return set_error(HL_EINVAL, "model: null pointer");
  if (m->n_layer <= 0 || m->n_emb <= 0 || m->n_head <= 0 || m->n_head_kv <= 0 || m->head_dim <= 0 ||
      m->n_ff <= 0 || m->n_vocab <= 0 || m->max_len <= 0)
    return set_error(HL_EINVAL, "model: bad shape");
  if (m->n_head % m->n_head_kv) return set_error(HL_EINVAL, "GQA requires head_count divisible by head_count_kv");
  const int rd = rope_dim_of(m);
  if ((rd & 1) || rd > m->head_dim)
    return set_error(HL_EINVAL, "model: rope_dim %d must be even and <= head_dim %d", rd, m->head_dim);
  if (!(m->rms_eps >= 0.f)) return set_error(HL_EINVAL, "model: rms_eps must be >= 0");
  const int E = m->n_emb, qdim = m->n_head * m->head_dim;
  for (int l = 0; l < m->n_layer; ++l) {
    const hl_layer_desc& L = m->layers[l];
    if (!L.attn_norm || !L.ffn_norm) return set_error(HL_EINVAL, "model: layer %d norm weight is null", l);
    int rc;
    if ((rc = check_weight(L.wq, L.wq_type, E, "wq", l, fp32_only)) ||
        (rc = check_weight(L.wk, L.wk_type, E, "wk", l, fp32_only)) ||
        (rc = check_weight(L.wv, L.wv_type, E, "wv", l, fp32_only)) ||
        (rc = check_weight(L.wo, L.wo_type, qdim, "wo", l, fp32_only)) ||
        (rc = check_weight(L.w_gate, L.w_gate_type, E, "w_gate", l, fp32_only)) ||
        (rc = check_weight(L.w_up, L.w_up_type, E, "w_up", l, fp32_only)) ||
        (rc = check_weight(L.w_down, L.w_down_type, m->n_ff, "w_down", l, fp32_only)))
      return rc;
  }
  return check_weight(m->output, m->output_type, E, "output", -1, fp32_only);
}

// y[rows, T] = W[rows, cols] . x[cols, T]: gpuLinearCol (fp32) or, for one
// column, gpuLinearColQuant.
static int linear_t(float* y, const float* x, const void* w, int type, int cols, int rows, int T, void* stream) {
  return type == 0 ? hl_gpu_linear_col(y, x, (const float*)w, cols, rows, T, stream)
                   : hl_gpu_linear_col_quant(y, x, w, cols, rows, type, stream);
}

// Quantized K/V (or gate/up) of one type as one launch where the direct
// kernel takes them (the reference's fused GEMVs); false: run them apart.
static bool pair_launch(int which, float* d0, float* d1, const float* x, const void* wa, const void* wb, int ta,
                        int tb, int cols, int rows, void* stream) {
  return ta != 0 && ta == tb && pair_fusable(ta, cols) &&
         linear_quant_pair_launch(which, d0, d1, x, wa, wb, cols, rows, ta, (hipStream_t)stream);
}

// Quantized Q, K and V of one type as one launch (the direct kernel's
// three-matrix mode); false: run Q, then the K/V pair.
static bool qkv_launch(float* q, float* k, float* v, const float* x, const hl_layer_desc& L, int cols, int qrows,
                       int kvrows, void* stream) {
  return L.wq_type != 0 && L.wq_type == L.wk_type && L.wq_type == L.wv_type && pair_fusable(L.wq_type, cols) &&
         linear_quant_qkv_launch(q, k, v, x, L.wq, L.wk, L.wv, cols, qrows, kvrows, L.wq_type, (hipStream_t)stream);
}

#define HL_TRY(call)              \
  do {                            \
    const int rc_ = (call);       \
    if (rc_ != HL_OK) return rc_; \
  } while (0)

// The FFN half of a decode layer after attention's O projection in tmp0:
// residual + ffn norm, gate/up, SiLU * up, down, residual + the next
// layer's norm (or the plain residual after the last layer).
static int decode_ffn(const hl_model_desc* m, int l, float* x, float* x_norm, float* tmp0, float* tmp1, float* tmp2,
                      void* stream) {
  const hl_layer_desc& L = m->layers[l];
  const int E = m->n_emb;
  const float eps = m->rms_eps;
  // Q4_K gate/up on the matrix cores takes the residual + norm into its own
  // x prologue; the sum then sits in x_norm until the next residual moves it
  // back to x.
  const bool folded = L.w_gate_type == L.w_up_type &&
                      linear_quant_gate_up_norm_launch(tmp2, x_norm, x, tmp0, L.ffn_norm, eps, L.w_gate, L.w_up, E,
                                                       m->n_ff, L.w_gate_type, (hipStream_t)stream);
  if (folded) {
    if (hipGetLastError() != hipSuccess) return set_error(HL_EHIP, "fused norm gate/up launch failed");
  } else {
    HL_TRY(hl_gpu_residual_rmsnorm(x_norm, x, tmp0, L.ffn_norm, E, eps, stream));
    if (!pair_launch(1, tmp2, nullptr, x_norm, L.w_gate, L.w_up, L.w_gate_type, L.w_up_type, E, m->n_ff, stream)) {
      HL_TRY(linear_t(tmp0, x_norm, L.w_gate, L.w_gate_type, E, m->n_ff, 1, stream));
      HL_TRY(linear_t(tmp1, x_norm, L.w_up, L.w_up_type, E, m->n_ff, 1, stream));
      HL_TRY(hl_gpu_silu_mul(tmp2, tmp0, tmp1, m->n_ff, stream));
    }
  }
  HL_TRY(linear_t(tmp0, tmp2, L.w_down, L.w_down_type, m->n_ff, E, 1, stream));
  const float* xs = folded ? x_norm : x;  // the residual stream
  if (l + 1 < m->n_layer) {
    if (residual_rmsnorm_from_launch(x_norm, x, xs, tmp0, m->layers[l + 1].attn_norm, E, eps, (hipStream_t)stream) !=
        hipSuccess)
      return set_error(HL_EHIP, "residual rmsnorm launch failed");
    return HL_OK;
  }
  return hl_gpu_add(x, xs, tmp0, E, stream);
}

// The gpuAttentionDecode call of the reference's step for layer l (fp32
// caches of the model descriptor).
static void dropin_args(hl_decode_args& a, const hl_model_desc* m, int l, const float* q, float* out, int L) {
  memset(&a, 0, sizeof(a));
  a.batch = 1;
  a.n_head = m->n_head;
  a.n_head_kv = m->n_head_kv;
  a.head_dim = m->head_dim;
  a.kv_dtype = HL_F32;
  a.max_len = m->max_len;
  a.seq_len = L;
  a.q = q;
  a.k_cache = m->layers[l].k_cache;
  a.v_cache = m->layers[l].v_cache;
  a.out = out;
}

int hl_forward_decode_token(const hl_model_desc* m, const hl_decode_scratch* s,
                            const int32_t* token_dev, int pos, float* logits,
                            int32_t* next_token_dev, void* stream) {
  if (!s || !token_dev || !logits || !next_token_dev || !s->x || !s->x_norm || !s->tmp0 || !s->tmp1 || !s->tmp2)
    return set_error(HL_EINVAL, "forward_decode_token: null pointer");
  HL_TRY(check_model(m, false));
  if (pos < 0 || pos >= m->max_len)
    return set_error(HL_ECAPACITY, "forward_decode_token: position %d outside the cache (%d)", pos,
                   m->max_len);
  for (int l = 0; l < m->n_layer; ++l) {
    if (!m->layers[l].k_cache || !m->layers[l].v_cache)
      return set_error(HL_EINVAL, "forward_decode_token: layer %d cache is null", l);
    hl_decode_args a;
    dropin_args(a, m, l, s->tmp0, s->x_norm, pos + 1);
    HL_TRY(check_decode_args(&a));
  }
  const int E = m->n_emb, D = m->head_dim, qdim = m->n_head * D, kvdim = m->n_head_kv * D;
  const int rd = rope_dim_of(m);
  const float eps = m->rms_eps;
  HL_TRY(hl_set_rope_theta(rd, m->rope_base));
  HL_TRY(hl_gpu_embedding(s->x, m->tok_emb, token_dev, E, 1, m->n_vocab, stream));
  HL_TRY(hl_gpu_rmsnorm_cols(s->x_norm, s->x, m->layers[0].attn_norm, E, 1, eps, stream));
  for (int l = 0; l < m->n_layer; ++l) {
    const hl_layer_desc& L = m->layers[l];
    if (!qkv_launch(s->tmp0, s->tmp1, s->tmp2, s->x_norm, L, E, qdim, kvdim, stream)) {
      HL_TRY(linear_t(s->tmp0, s->x_norm, L.wq, L.wq_type, E, qdim, 1, stream));
      if (!pair_launch(2, s->tmp1, s->tmp2, s->x_norm, L.wk, L.wv, L.wk_type, L.wv_type, E, kvdim, stream)) {
        HL_TRY(linear_t(s->tmp1, s->x_norm, L.wk, L.wk_type, E, kvdim, 1, stream));
        HL_TRY(linear_t(s->tmp2, s->x_norm, L.wv, L.wv_type, E, kvdim, 1, stream));
      }
    }
    if (L.q_norm) HL_TRY(hl_gpu_qk_norm(s->tmp0, L.q_norm, m->n_head, D, eps, stream));
    if (L.k_norm) HL_TRY(hl_gpu_qk_norm(s->tmp1, L.k_norm, m->n_head_kv, D, eps, stream));
    HL_TRY(hl_gpu_rope_qk_decode(s->tmp0, s->tmp1, m->n_head, m->n_head_kv, D, rd, m->rope_base, pos, stream));
    HL_TRY(hl_gpu_store_kv_pair(L.k_cache, s->tmp1, L.v_cache, s->tmp2, kvdim, 1, m->max_len, pos, stream));
    HL_TRY(hl_gpu_attention_decode(s->x_norm, s->tmp0, L.k_cache, L.v_cache, m->n_head, m->n_head_kv,
                                   D, pos + 1, m->max_len, stream));
    HL_TRY(linear_t(s->tmp0, s->x_norm, L.wo, L.wo_type, qdim, E, 1, stream));
    HL_TRY(decode_ffn(m, l, s->x, s->x_norm, s->tmp0, s->tmp1, s->tmp2, stream));
  }
  HL_TRY(hl_gpu_rmsnorm_cols(s->x_norm, s->x, m->output_norm, E, 1, eps, stream));
  HL_TRY(linear_t(logits, s->x_norm, m->output, m->output_type, E, m->n_vocab, 1, stream));
  return hl_argmax_async(logits, m->n_vocab, next_token_dev, stream);
}

// ---------------------------------------------------------------------------
// KV-cache descriptor, prefill and decode over it
// ---------------------------------------------------------------------------
static int elem_bytes(int dt) { return dt == HL_F32 ? 4 : (dt == HL_FP8 ? 1 : 2); }

size_t hl_kv_cache_bytes(int n_head_kv, int head_dim, int max_len, int kv_dtype, int kv_layout) {
  if (n_head_kv <= 0 || head_dim <= 0 || max_len <= 0) return 0;
  if (kv_dtype != HL_F32 && kv_dtype != HL_F16 && kv_dtype != HL_BF16 && kv_dtype != HL_FP8) return 0;
  if (kv_layout == HL_KV_COLMAJOR) {
    if (kv_dtype == HL_FP8) return 0;
  } else if (kv_layout == HL_KV_TILED32 || kv_layout == HL_KV_PAGED32) {
    if (kv_dtype == HL_F32 || max_len % 32) return 0;
  } else {
    return 0;
  }
  return (size_t)n_head_kv * head_dim * max_len * elem_bytes(kv_dtype);
}

int hl_kv_cache_preferred_layout(int kv_dtype, int max_len) {
  const bool tiles = (kv_dtype == HL_F16 || kv_dtype == HL_BF16 || kv_dtype == HL_FP8) && max_len > 0 &&
                     max_len % 32 == 0;
  return tiles ? HL_KV_TILED32 : HL_KV_COLMAJOR;
}

// The decode step's calls for layer l at position pos (q, k, v: the new
// token's projections; out: the attention output).
static void step_args(hl_rope_store_args& r, hl_decode_args& a, const hl_model_desc* m, const hl_kv_cache_desc* c,
                      int l, float* q, float* k, const float* v, float* out, int pos) {
  memset(&r, 0, sizeof(r));
  r.batch = 1;
  r.n_head_q = m->n_head;
  r.n_head_kv = m->n_head_kv;
  r.head_dim = m->head_dim;
  r.rope_dim = rope_dim_of(m);
  r.rope_style = HL_ROPE_HALF_SPLIT;
  r.rope_base = m->rope_base;
  r.kv_dtype = c->kv_dtype;
  r.max_len = c->max_len;
  r.q = q;
  r.k = k;
  r.v = v;
  r.k_cache = c->k[l];
  r.v_cache = c->v[l];
  r.pos = pos;
  r.q_norm_w = m->layers[l].q_norm;
  r.k_norm_w = m->layers[l].k_norm;
  r.eps = m->rms_eps;
  r.kv_layout = c->kv_layout;
  r.block_table = c->block_table;
  r.blocks_per_seq = c->blocks_per_seq;
  memset(&a, 0, sizeof(a));
  a.batch = 1;
  a.n_head = m->n_head;
  a.n_head_kv = m->n_head_kv;
  a.head_dim = m->head_dim;
  a.kv_dtype = c->kv_dtype;
  a.max_len = c->max_len;
  a.seq_len = pos + 1;
  a.q = q;
  a.k_cache = c->k[l];
  a.v_cache = c->v[l];
  a.out = out;
  a.kv_layout = c->kv_layout;
  a.block_table = c->block_table;
  a.blocks_per_seq = c->blocks_per_seq;
}

// The prefill attention call for layer l over T tokens: q/k/v projections
// in, qk-norm + RoPE + cache write + causal attention, output into out.
static void prefill_args(hl_prefill_args& p, const hl_model_desc* m, const hl_kv_cache_desc* c, int l,
                         const float* q, const float* k, const float* v, float* out, int T) {
  memset(&p, 0, sizeof(p));
  p.n_head = m->n_head;
  p.n_head_kv = m->n_head_kv;
  p.head_dim = m->head_dim;
  p.seq_len = T;
  p.io_dtype = HL_F32;
  p.q = q;
  p.k = k;
  p.v = v;
  p.out = out;
  p.q_norm_w = m->layers[l].q_norm;
  p.k_norm_w = m->layers[l].k_norm;
  p.eps = m->rms_eps;
  p.apply_rope = 1;
  p.rope_dim = rope_dim_of(m);
  p.rope_style = HL_ROPE_HALF_SPLIT;
  p.rope_base = m->rope_base;
  p.k_cache = c->k[l];
  p.v_cache = c->v[l];
  p.kv_dtype = c->kv_dtype;
  p.max_len = c->max_len;
  p.start_pos = 0;
  p.out_dtype = HL_F32;
  p.kv_layout = c->kv_layout;
  p.block_table = c->block_table;
}

static int check_cache(const hl_kv_cache_desc* c, const hl_model_desc* m) {
  if (!c || !c->k || !c->v) return set_error(HL_EINVAL, "kv cache: null pointer");
  if (c->n_layer != m->n_layer || c->n_head_kv != m->n_head_kv || c->head_dim != m->head_dim)
    return set_error(HL_EINVAL, "kv cache: shape (%d layers, %d kv heads, dim %d) does not match the model "
                                "(%d, %d, %d)", c->n_layer, c->n_head_kv, c->head_dim, m->n_layer,
                     m->n_head_kv, m->head_dim);
  if (c->max_len <= 0) return set_error(HL_EINVAL, "kv cache: max_len must be >= 1");
  if (!hl_kv_cache_bytes(c->n_head_kv, c->head_dim, c->max_len, c->kv_dtype, c->kv_layout))
    return set_error(HL_EUNSUPPORTED, "kv cache: dtype %d with layout %d (max_len %d) is not built",
                     c->kv_dtype, c->kv_layout, c->max_len);
  for (int l = 0; l < c->n_layer; ++l)
    if (!c->k[l] || !c->v[l]) return set_error(HL_EINVAL, "kv cache: layer %d cache is null", l);
  if (c->cur_len < 0 || c->cur_len > c->max_len) return set_error(HL_EINVAL, "kv cache: cur_len %d outside [0, %d]", c->cur_len, c->max_len);
  return HL_OK;
}

int hl_kv_cache_init(hl_kv_cache_desc* c, const hl_model_desc* m) {
  HL_TRY(check_model(m, false));
  if (!c) return set_error(HL_EINVAL, "kv cache: null pointer");
  c->cur_len = 0;
  HL_TRY(check_cache(c, m));
  // every layer's decode-step call at the last position (dtype, layout,
  // alignment, block table and head-dim rules of the attention entry points)
  float* fake = (float*)(uintptr_t)256;  // stands in for the activations; never dereferenced here
  for (int l = 0; l < c->n_layer; ++l) {
    hl_rope_store_args r;
    hl_decode_args a;
    step_args(r, a, m, c, l, fake, fake, fake, fake, c->max_len - 1);
    HL_TRY(check_step_args(&r, &a));
  }
  return HL_OK;
}

static int check_scratch(const hl_forward_scratch* s, int T) {
  if (!s || !s->x || !s->x_norm || !s->tmp0 || !s->tmp1 || !s->tmp2)
    return set_error(HL_EINVAL, "forward: scratch has a null buffer");
  if (s->max_tokens < T)
    return set_error(HL_EINVAL, "forward: scratch holds %d tokens, %d needed", s->max_tokens, T);
  return HL_OK;
}

// The forward workspace: the decode steps' split-K region first (its
// arrival counters stay zero between steps), the prefill's operand region
// after it.  The decode region is bounded in closed form: the counters of
// the smallest head chunks and at most min(256, tiles of max_len) splits of
// (head_dim + 2) floats per query head (the decode plan's limits).
static size_t decode_region_bytes(const hl_model_desc* m, const hl_kv_cache_desc* c) {
  const long long G = m->n_head / m->n_head_kv;
  const long long chunks = G;
  const size_t counters = ((size_t)m->n_head_kv * chunks * 4 + 255) / 256 * 256;
  const long long tiles = (c->max_len + 31) / 32;
  const long long S = tiles < 256 ? tiles : 256;
  const size_t partials = (size_t)m->n_head * S * (m->head_dim + 2) * 4;
  return (counters + partials + 255) / 256 * 256;
}

size_t hl_forward_workspace_bytes(const hl_model_desc* m, const hl_kv_cache_desc* c, int max_tokens) {
  if (check_model(m, false) || check_cache(c, m) || max_tokens < 1) return 0;
  float* fake = (float*)(uintptr_t)256;  // stands in for the activations; never dereferenced here
  hl_prefill_args p;
  prefill_args(p, m, c, 0, fake, fake, fake, fake, max_tokens < c->max_len ? max_tokens : c->max_len);
  return decode_region_bytes(m, c) + hl_attn_prefill_workspace_bytes(&p);
}

static int check_workspace(const hl_forward_scratch* s, size_t need) {
  if (need == 0) return HL_OK;
  if (!s->workspace || s->workspace_bytes < need)
    return set_error(HL_EINVAL, "forward: attention workspace of %zu bytes needed, %zu given", need,
                     s->workspace_bytes);
  if ((uintptr_t)s->workspace & 15) return set_error(HL_EINVAL, "forward: workspace must be 16-byte aligned");
  return HL_OK;
}

int hl_forward_prefill(const hl_model_desc* m, hl_kv_cache_desc* c, const hl_forward_scratch* s,
                       const int32_t* tokens_dev, int T, float* logits, void* stream) {
  HL_TRY(check_model(m, true));
  HL_TRY(check_cache(c, m));
  if (T <= 0) return set_error(HL_EINVAL, "prefill requires at least one token");
  if (T > c->max_len) return set_error(HL_ECAPACITY, "prefill exceeds KV cache capacity");
  if (!tokens_dev || !logits) return set_error(HL_EINVAL, "prefill: null pointer");
  HL_TRY(check_scratch(s, T));
  const size_t dec = decode_region_bytes(m, c);
  size_t need = 0;
  for (int l = 0; l < m->n_layer; ++l) {
    hl_prefill_args p;
    prefill_args(p, m, c, l, s->tmp0, s->tmp1, s->tmp2, s->x_norm, T);
    HL_TRY(check_prefill_args(&p));
    const size_t b = hl_attn_prefill_workspace_bytes(&p);
    if (b > need) need = b;
  }
  HL_TRY(check_workspace(s, dec + need));
  void* pws = (char*)s->workspace + dec;  // the prefill never touches the decode region
  const size_t pws_bytes = s->workspace_bytes - dec;

  const int E = m->n_emb, qdim = m->n_head * m->head_dim, kvdim = m->n_head_kv * m->head_dim;
  const float eps = m->rms_eps;
  float *x = s->x, *xn = s->x_norm, *t0 = s->tmp0, *t1 = s->tmp1, *t2 = s->tmp2;
  HL_TRY(hl_gpu_embedding(x, m->tok_emb, tokens_dev, E, T, m->n_vocab, stream));
  for (int l = 0; l < m->n_layer; ++l) {
    const hl_layer_desc& L = m->layers[l];
    HL_TRY(hl_gpu_rmsnorm_cols(xn, x, L.attn_norm, E, T, eps, stream));
    HL_TRY(hl_gpu_linear_col(t0, xn, (const float*)L.wq, E, qdim, T, stream));
    HL_TRY(hl_gpu_linear_col(t1, xn, (const float*)L.wk, E, kvdim, T, stream));
    HL_TRY(hl_gpu_linear_col(t2, xn, (const float*)L.wv, E, kvdim, T, stream));
    // qk-norm, RoPE at positions 0 .. T-1, the cache write of columns
    // 0 .. T-1 and causal attention (naive.nim:4066-4078) in one call
    hl_prefill_args p;
    prefill_args(p, m, c, l, t0, t1, t2, xn, T);
    HL_TRY(hl_attn_prefill(&p, pws, pws_bytes, stream));
    HL_TRY(hl_gpu_linear_col(t0, xn, (const float*)L.wo, qdim, E, T, stream));
    HL_TRY(hl_gpu_add(x, x, t0, E * T, stream));
    HL_TRY(hl_gpu_rmsnorm_cols(xn, x, L.ffn_norm, E, T, eps, stream));
    HL_TRY(hl_gpu_linear_col(t0, xn, (const float*)L.w_gate, E, m->n_ff, T, stream));
    HL_TRY(hl_gpu_linear_col(t1, xn, (const float*)L.w_up, E, m->n_ff, T, stream));
    HL_TRY(hl_gpu_silu_mul(t2, t0, t1, m->n_ff * T, stream));
    HL_TRY(hl_gpu_linear_col(t0, t2, (const float*)L.w_down, m->n_ff, E, T, stream));
    HL_TRY(hl_gpu_add(x, x, t0, E * T, stream));
  }
  HL_TRY(hl_gpu_rmsnorm_cols(xn, x, m->output_norm, E, T, eps, stream));
  HL_TRY(hl_gpu_linear_col(logits, xn, (const float*)m->output, E, m->n_vocab, T, stream));
  c->cur_len = T;
  return HL_OK;
}

int hl_forward_decode(const hl_model_desc* m, hl_kv_cache_desc* c, const hl_forward_scratch* s,
                      const int32_t* token_dev, float* logits, int32_t* next_token_dev, void* stream) {
  HL_TRY(check_model(m, false));
  HL_TRY(check_cache(c, m));
  if (!token_dev || !logits || !next_token_dev) return set_error(HL_EINVAL, "forward_decode: null pointer");
  HL_TRY(check_scratch(s, 1));
  const int pos = c->cur_len;
  if (pos >= c->max_len) return set_error(HL_ECAPACITY, "KV cache full");
  for (int l = 0; l < m->n_layer; ++l) {
    hl_rope_store_args r;
    hl_decode_args a;
    step_args(r, a, m, c, l, s->tmp0, s->tmp1, s->tmp2, s->x_norm, pos);
    HL_TRY(check_step_args(&r, &a));
  }
  HL_TRY(check_workspace(s, decode_region_bytes(m, c)));

  const int E = m->n_emb, qdim = m->n_head * m->head_dim, kvdim = m->n_head_kv * m->head_dim;
  const float eps = m->rms_eps;
  HL_TRY(hl_gpu_embedding(s->x, m->tok_emb, token_dev, E, 1, m->n_vocab, stream));
  HL_TRY(hl_gpu_rmsnorm_cols(s->x_norm, s->x, m->layers[0].attn_norm, E, 1, eps, stream));
  for (int l = 0; l < m->n_layer; ++l) {
    const hl_layer_desc& L = m->layers[l];
    if (!qkv_launch(s->tmp0, s->tmp1, s->tmp2, s->x_norm, L, E, qdim, kvdim, stream)) {
      HL_TRY(linear_t(s->tmp0, s->x_norm, L.wq, L.wq_type, E, qdim, 1, stream));
      if (!pair_launch(2, s->tmp1, s->tmp2, s->x_norm, L.wk, L.wv, L.wk_type, L.wv_type, E, kvdim, stream)) {
        HL_TRY(linear_t(s->tmp1, s->x_norm, L.wk, L.wk_type, E, kvdim, 1, stream));
        HL_TRY(linear_t(s->tmp2, s->x_norm, L.wv, L.wv_type, E, kvdim, 1, stream));
      }
    }
    // qk-norm + RoPE + the cache write at pos + attention over pos + 1
    // columns (naive.nim:4697-4717): one launch for fp16/bf16/fp8 caches
    hl_rope_store_args r;
    hl_decode_args a;
    step_args(r, a, m, c, l, s->tmp0, s->tmp1, s->tmp2, s->x_norm, pos);
    HL_TRY(hl_decode_step(&r, &a, s->workspace, decode_region_bytes(m, c), stream));
    HL_TRY(linear_t(s->tmp0, s->x_norm, L.wo, L.wo_type, qdim, E, 1, stream));
    HL_TRY(decode_ffn(m, l, s->x, s->x_norm, s->tmp0, s->tmp1, s->tmp2, stream));
  }
  HL_TRY(hl_gpu_rmsnorm_cols(s->x_norm, s->x, m->output_norm, E, 1, eps, stream));
  HL_TRY(linear_t(logits, s->x_norm, m->output, m->output_type, E, m->n_vocab, 1, stream));
  HL_TRY(hl_argmax_async(logits, m->n_vocab, next_token_dev, stream));
  c->cur_len = pos + 1;
  return HL_OK;
}

}  // extern "C"

namespace {
// The two timing events of hl_forward_decode_timed, created on first use per
// device and kept for the process (forwardDecodeTokenTimed's module-level
// mkBenchEvent0/1, megakernel.nim:2516-2519).
constexpr int kMaxDevices = 64;
std::mutex g_ev_mu;
hipEvent_t g_ev[kMaxDevices][2];

int timing_events(hipEvent_t& e0, hipEvent_t& e1) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(HL_EHIP, "forward_decode_timed: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error(HL_EUNSUPPORTED, "forward_decode_timed: device %d", dev);
  std::lock_guard<std::mutex> lk(g_ev_mu);
  for (int i = 0; i < 2; ++i)
    if (!g_ev[dev][i] && (e = hipEventCreate(&g_ev[dev][i])) != hipSuccess)
      return set_error(HL_EHIP, "forward_decode_timed: hipEventCreate: %s", hipGetErrorString(e));
  e0 = g_ev[dev][0];
  e1 = g_ev[dev][1];
  return HL_OK;
}
}  // namespace

extern "C" {

int hl_forward_decode_timed(const hl_model_desc* m, hl_kv_cache_desc* c, const hl_forward_scratch* s,
                            const int32_t* token_dev, float* logits, int32_t* next_token_dev,
                            int32_t* next_token, float* gpu_ms, void* stream) {
  if (!next_token || !gpu_ms) return set_error(HL_EINVAL, "forward_decode_timed: null pointer");
  const hipStream_t st = (hipStream_t)stream;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(st, &cs);
  if (e != hipSuccess) return set_error(HL_EHIP, "hipStreamIsCapturing: %s", hipGetErrorString(e));
  if (cs != hipStreamCaptureStatusNone)
    return set_error(HL_ECAPTURE, "forward_decode_timed waits for the stream; it cannot run under stream capture");
  hipEvent_t e0, e1;
  HL_TRY(timing_events(e0, e1));
  if ((e = hipEventRecord(e0, st)) != hipSuccess)
    return set_error(HL_EHIP, "forward_decode_timed: event record: %s", hipGetErrorString(e));
  HL_TRY(hl_forward_decode(m, c, s, token_dev, logits, next_token_dev, stream));
  if ((e = hipEventRecord(e1, st)) != hipSuccess)
    return set_error(HL_EHIP, "forward_decode_timed: event record: %s", hipGetErrorString(e));
  if ((e = hipMemcpyAsync(next_token, next_token_dev, sizeof(int32_t), hipMemcpyDeviceToHost, st)) != hipSuccess)
    return set_error(HL_EHIP, "forward_decode_timed: token copy: %s", hipGetErrorString(e));
  if ((e = hipStreamSynchronize(st)) != hipSuccess)
    return set_error(HL_EHIP, "forward_decode_timed: sync: %s", hipGetErrorString(e));
  if ((e = hipEventElapsedTime(gpu_ms, e0, e1)) != hipSuccess)
    return set_error(HL_EHIP, "forward_decode_timed: elapsed time: %s", hipGetErrorString(e));
  return HL_OK;
}

}  // extern "C"
