// C ABI of libhl_attn.so: argument checks, workspace planning and dispatch.
//
// Error behaviour mirrors the reference's host prechecks, which raise
// ValueError with these messages (backends/naive.nim):
//   "GQA requires head_count divisible by head_count_kv"   :3971-3972, 4596-4597
//   "prefill requires at least one token"                   :3973-3974
//   "prefill exceeds KV cache capacity"                     :3975-3976
//   "KV cache full"                                         :4598-4599
// Each becomes a negative status plus the same text from hl_last_error().
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "common.h"
#include "launch.h"

using namespace hl;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(HL_EHIP, "%s: %s", what, hipGetErrorString(e));
}

inline hipStream_t as_stream(void* s) { return (hipStream_t)s; }

}  // namespace

// The thread's error message for entry points in other translation units.
int hl::set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

namespace {

std::mutex g_mu;
bool g_theta_set = false;
int g_theta_dim = 0;
ThetaTable g_theta;

// Library-owned split-K workspace for the reference-signature decode entry
// point (the reference keeps such scratch in its module-global GpuContext).
struct DevWs {
  void* ptr = nullptr;
  size_t bytes = 0;
  size_t zero_prefix = 0;  // leading bytes known to hold zero arrival counters
};
std::vector<DevWs> g_ws;
// The same for the reference-signature prefill entry point (its fp32 K/V
// split images); grown on demand, per device.
std::vector<DevWs> g_pws;
std::vector<void*> g_argmax_ws;  // per device, kArgmaxScratchBytes, counter zero between calls

void build_theta(ThetaTable& t, int rope_dim, float base) {
  memset(&t, 0, sizeof(t));
  for (int i = 0; i < rope_dim / 2; ++i)
    t.t[i] = powf(1.0f / base, (2.0f * (float)i) / (float)rope_dim);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The library-owned scratch of the reference-signature drop-ins is allocated
// (with a device synchronisation) when a call first needs it; that cannot
// happen inside a HIP graph capture, so such a call is refused instead.
int refuse_if_capturing(void* stream, const char* what) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(as_stream(stream), &st);
  if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
  if (st != hipStreamCaptureStatusNone)
    return fail(HL_ECAPTURE, "%s: the first call of this size on a device allocates; it cannot run under stream capture (call once before capturing)", what);
  return HL_OK;
}

int check_gqa(int n_head, int n_head_kv) {
  if (n_head <= 0 || n_head_kv <= 0)
    return fail(HL_EINVAL, "head counts must be positive (n_head=%d, n_head_kv=%d)", n_head, n_head_kv);
  if (n_head % n_head_kv != 0)
    return fail(HL_EINVAL, "GQA requires head_count divisible by head_count_kv");
  return HL_OK;
}

int check_dtype(int dt, const char* what) {
  if (dt != HL_F32 && dt != HL_F16 && dt != HL_BF16)
    return fail(HL_EINVAL, "%s: unknown dtype %d", what, dt);
  return HL_OK;
}

// KV caches may also be fp8 (tiled layout only, checked with the layout).
int check_kv_dtype(int dt, const char* what) {
  return dt == HL_FP8 ? HL_OK : check_dtype(dt, what);
}

int check_rope(int head_dim, int rope_dim, int style) {
  if (rope_dim <= 0 || rope_dim > head_dim || (rope_dim & 1) || rope_dim > HL_MAX_ROPE_DIM)
    return fail(HL_EINVAL, "rope_dim %d must be even and in [2, head_dim=%d]", rope_dim, head_dim);
  if (style != HL_ROPE_HALF_SPLIT && style != HL_ROPE_INTERLEAVED)
    return fail(HL_EINVAL, "unknown rope_style %d", style);
  return HL_OK;
}

// Theta for an op: installed table (must match rope_dim) or built from base.
int theta_for(int use_installed, int rope_dim, float base, ThetaTable& out) {
  if (use_installed) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_theta_set) return fail(HL_EINVAL, "no RoPE theta table installed (hl_set_rope_theta)");
    if (g_theta_dim != rope_dim)
      return fail(HL_EINVAL, "installed theta table has rope_dim %d, call uses %d", g_theta_dim, rope_dim);
    out = g_theta;
    return HL_OK;
  }
  if (!(base > 0.f)) return fail(HL_EINVAL, "rope_base must be > 0");
  build_theta(out, rope_dim, base);
  return HL_OK;
}

}  // namespace

extern "C" {

const char* hl_last_error(void) { return g_err; }

int hl_abi_version(void) { return 3; }  // 2: kv_layout in the args; 3: block_table (paged caches)

int hl_device_info_get(hl_device_info* info) {
  if (!info) return fail(HL_EINVAL, "info is null");
  memset(info, 0, sizeof(*info));
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  hipDeviceProp_t pr;
  e = hipGetDeviceProperties(&pr, dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  info->device = dev;
  info->cu_count = pr.multiProcessorCount;
  info->clock_khz = pr.clockRate;
  info->mem_clock_khz = pr.memoryClockRate;
  info->l2_bytes = pr.l2CacheSize;
  info->hbm_bytes = pr.totalGlobalMem;
  info->hbm_peak_gbs = 8000.0;
  info->bf16_dense_tflops = (double)pr.multiProcessorCount * (pr.clockRate * 1e3) * 4096.0 / 1e12;
  info->fp32_tflops = 157.3;
  strncpy(info->arch, pr.gcnArchName, sizeof(info->arch) - 1);
  return HL_OK;
}

int hl_rope_theta_table(float* theta_out, int rope_dim, float rope_base) {
  if (!theta_out) return fail(HL_EINVAL, "theta_out is null");
  if (rope_dim <= 0 || (rope_dim & 1) || rope_dim > HL_MAX_ROPE_DIM)
    return fail(HL_EINVAL, "rope_dim %d must be even and <= %d", rope_dim, HL_MAX_ROPE_DIM);
  if (!(rope_base > 0.f)) return fail(HL_EINVAL, "rope_base must be > 0");
  ThetaTable t;
  build_theta(t, rope_dim, rope_base);
  memcpy(theta_out, t.t, sizeof(float) * (rope_dim / 2));
  return HL_OK;
}

int hl_set_rope_theta(int rope_dim, float rope_base) {
  if (rope_dim <= 0 || (rope_dim & 1) || rope_dim > HL_MAX_ROPE_DIM)
    return fail(HL_EINVAL, "rope_dim %d must be even and <= %d", rope_dim, HL_MAX_ROPE_DIM);
  if (!(rope_base > 0.f)) return fail(HL_EINVAL, "rope_base must be > 0");
  std::lock_guard<std::mutex> lk(g_mu);
  build_theta(g_theta, rope_dim, rope_base);
  g_theta_dim = rope_dim;
  g_theta_set = true;
  return HL_OK;
}

// ---------------------------------------------------------------------------
// Reference-signature drop-ins
// ---------------------------------------------------------------------------
int hl_gpu_qk_norm(float* x, const float* weight, int n_head, int head_dim, float eps,
                   void* stream) {
  if (!x || !weight) return fail(HL_EINVAL, "qk_norm: null pointer");
  if (n_head <= 0 || head_dim <= 0 || head_dim > HL_MAX_HEAD_DIM)
    return fail(HL_EINVAL, "qk_norm: bad shape n_head=%d head_dim=%d", n_head, head_dim);
  HeadVecOp op;
  memset(&op, 0, sizeof(op));
  op.q = x;
  op.q_norm_w = weight;
  op.eps = eps;
  op.batch = 1;
  op.n_head_q = n_head;
  op.head_dim = head_dim;
  op.rope_dim = 0;
  hipError_t e = headvec_launch(op, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "qk_norm launch");
}

int hl_gpu_qk_norm_prefill(float* x, const float* weight, int n_head, int head_dim, int seq_len,
                           float eps, void* stream) {
  if (!x || !weight) return fail(HL_EINVAL, "qk_norm_prefill: null pointer");
  if (n_head <= 0 || head_dim <= 0 || head_dim > HL_MAX_HEAD_DIM || seq_len <= 0)
    return fail(HL_EINVAL, "qk_norm_prefill: bad shape");
  PrologueOp op;
  memset(&op, 0, sizeof(op));
  op.q = x;
  op.q_inplace = x;
  op.io_dtype = HL_F32;
  op.q_norm_w = weight;
  op.eps = eps;
  op.n_head = n_head;
  op.n_head_kv = 0;
  op.head_dim = head_dim;
  op.seq_len = seq_len;
  op.t_pad = seq_len;
  op.kv_dtype = HL_F32;
  hipError_t e = prologue_launch(op, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "qk_norm_prefill launch");
}

static int rope_cols_common(float* x, int n_head, int head_dim, int rope_dim, int pos0,
                            int seq_len, const ThetaTable& th, void* stream) {
  PrologueOp op;
  memset(&op, 0, sizeof(op));
  op.q = x;
  op.q_inplace = x;
  op.io_dtype = HL_F32;
  op.n_head = n_head;
  op.head_dim = head_dim;
  op.seq_len = seq_len;
  op.t_pad = seq_len;
  op.do_rope = 1;
  op.rope_dim = rope_dim;
  op.rope_style = HL_ROPE_HALF_SPLIT;
  op.start_pos = pos0;
  op.kv_dtype = HL_F32;
  op.theta = th;
  hipError_t e = prologue_launch(op, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "rope launch");
}

static int rope_vec_common(float* q, float* k, int n_head_q, int n_head_k, int head_dim,
                           int rope_dim, int pos, const ThetaTable& th, void* stream) {
  HeadVecOp op;
  memset(&op, 0, sizeof(op));
  op.q = q;
  op.k = k;
  op.batch = 1;
  op.n_head_q = n_head_q;
  op.n_head_kv = k ? n_head_k : 0;
  op.head_dim = head_dim;
  op.rope_dim = rope_dim;
  op.rope_style = HL_ROPE_HALF_SPLIT;
  op.do_rope = 1;
  op.rope_q = 1;
  op.rope_k = 1;
  op.pos = pos;
  op.theta = th;
  hipError_t e = headvec_launch(op, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "rope launch");
}

int hl_gpu_rope_at_pos(float* x, int n_head, int head_dim, int rope_dim, float rope_base, int pos,
                       int seq_len, void* stream) {
  if (!x) return fail(HL_EINVAL, "rope_at_pos: null pointer");
  if (n_head <= 0 || head_dim <= 0 || head_dim > HL_MAX_HEAD_DIM || seq_len <= 0)
    return fail(HL_EINVAL, "rope_at_pos: bad shape");
  int rc = check_rope(head_dim, rope_dim, HL_ROPE_HALF_SPLIT);
  if (rc) return rc;
  ThetaTable th;
  if ((rc = theta_for(0, rope_dim, rope_base, th))) return rc;
  if (seq_len == 1) return rope_vec_common(x, nullptr, n_head, 0, head_dim, rope_dim, pos, th, stream);
  // seq_len > 1: column p rotated at position p (the reference ignores pos)
  return rope_cols_common(x, n_head, head_dim, rope_dim, 0, seq_len, th, stream);
}

int hl_gpu_rope_at_pos_theta(float* x, int n_head, int head_dim, int rope_dim, int pos,
                             int seq_len, void* stream) {
  if (!x) return fail(HL_EINVAL, "rope_at_pos_theta: null pointer");
  if (n_head <= 0 || head_dim <= 0 || head_dim > HL_MAX_HEAD_DIM || seq_len <= 0)
    return fail(HL_EINVAL, "rope_at_pos_theta: bad shape");
  int rc = check_rope(head_dim, rope_dim, HL_ROPE_HALF_SPLIT);
  if (rc) return rc;
  ThetaTable th;
  if ((rc = theta_for(1, rope_dim, 0.f, th))) return rc;
  if (seq_len == 1) return rope_vec_common(x, nullptr, n_head, 0, head_dim, rope_dim, pos, th, stream);
  return rope_cols_common(x, n_head, head_dim, rope_dim, pos, seq_len, th, stream);
}

int hl_gpu_rope_qk_decode(float* q, float* k, int n_head_q, int n_head_k, int head_dim,
                          int rope_dim, float rope_base, int pos, void* stream) {
  if (!q || !k) return fail(HL_EINVAL, "rope_qk_decode: null pointer");
  if (n_head_q <= 0 || n_head_k <= 0 || head_dim <= 0 || head_dim > HL_MAX_HEAD_DIM)
    return fail(HL_EINVAL, "rope_qk_decode: bad shape");
  int rc = check_rope(head_dim, rope_dim, HL_ROPE_HALF_SPLIT);
  if (rc) return rc;
  ThetaTable th;
  bool installed;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    installed = g_theta_set && g_theta_dim == rope_dim;
  }
  if ((rc = theta_for(installed ? 1 : 0, rope_dim, rope_base, th))) return rc;
  return rope_vec_common(q, k, n_head_q, n_head_k, head_dim, rope_dim, pos, th, stream);
}

int hl_gpu_fused_rope_store_kv(float* q, float* k, const float* v, float* k_cache, float* v_cache,
                               int n_head_q, int n_head_k, int head_dim, int rope_dim, int kv_dim,
                               int cache_cols, int pos, void* stream) {
  if (!q || !k || !v || !k_cache || !v_cache) return fail(HL_EINVAL, "fused_rope_store_kv: null pointer");
  if (n_head_q <= 0 || n_head_k <= 0 || head_dim <= 0 || head_dim > HL_MAX_HEAD_DIM)
    return fail(HL_EINVAL, "fused_rope_store_kv: bad shape");
  if (kv_dim != n_head_k * head_dim)
    return fail(HL_EINVAL, "fused_rope_store_kv: kv_dim %d != n_head_k*head_dim %d", kv_dim,
                n_head_k * head_dim);
  if (pos < 0 || pos >= cache_cols) return fail(HL_ECAPACITY, "KV cache full");
  int rc = check_rope(head_dim, rope_dim, HL_ROPE_HALF_SPLIT);
  if (rc) return rc;
  ThetaTable th;
  if ((rc = theta_for(1, rope_dim, 0.f, th))) return rc;
  HeadVecOp op;
  memset(&op, 0, sizeof(op));
  op.q = q;
  op.k = k;
  op.v = v;
  op.k_cache = k_cache;
  op.v_cache = v_cache;
  op.batch = 1;
  op.n_head_q = n_head_q;
  op.n_head_kv = n_head_k;
  op.head_dim = head_dim;
  op.rope_dim = rope_dim;
  op.rope_style = HL_ROPE_HALF_SPLIT;
  op.do_rope = 1;
  op.rope_q = 1;
  op.rope_k = 1;
  op.kv_dtype = HL_F32;
  op.max_len = cache_cols;
  op.batch_stride = (long long)kv_dim * cache_cols;
  op.pos = pos;
  op.theta = th;
  hipError_t e = headvec_launch(op, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "fused_rope_store_kv launch");
}

int hl_gpu_store_kv(float* cache, const float* src, int rows, int src_cols, int cache_cols,
                    int start_pos, void* stream) {
  if (!cache || !src) return fail(HL_EINVAL, "store_kv: null pointer");
  if (rows <= 0 || src_cols <= 0 || start_pos < 0) return fail(HL_EINVAL, "store_kv: bad shape");
  if (start_pos + src_cols > cache_cols) return fail(HL_ECAPACITY, "prefill exceeds KV cache capacity");
  hipError_t e = store_cols_launch(cache, src, nullptr, nullptr, rows, src_cols, cache_cols,
                                   start_pos, HL_F32, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "store_kv launch");
}

int hl_gpu_store_kv_pair(float* k_cache, const float* k_src, float* v_cache, const float* v_src,
                         int rows, int src_cols, int cache_cols, int start_pos, void* stream) {
  if (!k_cache || !k_src || !v_cache || !v_src) return fail(HL_EINVAL, "store_kv_pair: null pointer");
  if (rows <= 0 || src_cols <= 0 || start_pos < 0) return fail(HL_EINVAL, "store_kv_pair: bad shape");
  if (start_pos + src_cols > cache_cols) return fail(HL_ECAPACITY, "KV cache full");
  hipError_t e = store_cols_launch(k_cache, k_src, v_cache, v_src, rows, src_cols, cache_cols,
                                   start_pos, HL_F32, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "store_kv_pair launch");
}

// ---------------------------------------------------------------------------
// KV-cache layout
// ---------------------------------------------------------------------------
// Tiled and paged caches are read with vector loads of whole 32-column tile
// rows: fp16/bf16/fp8, whole tiles (max_len % 32), aligned sequences and
// caches; paged caches also need a block table covering max_len columns.
// fp8 caches exist only in those two layouts.
static int check_layout(int layout, int kv_dtype, int max_len, long long stride, const void* kc,
                        const void* vc, const void* table, int bps, const char* who) {
  if (layout == HL_KV_COLMAJOR) {
    if (kv_dtype == HL_FP8) return fail(HL_EUNSUPPORTED, "%s: fp8 KV caches need the tiled or paged layout", who);
    return HL_OK;
  }
  if (layout != HL_KV_TILED32 && layout != HL_KV_PAGED32)
    return fail(HL_EINVAL, "%s: unknown kv_layout %d", who, layout);
  if (kv_dtype == HL_F32)
    return fail(HL_EUNSUPPORTED, "%s: tiled and paged KV caches are fp16/bf16/fp8 only", who);
  if (max_len % 32)
    return fail(HL_EINVAL, "%s: tiled and paged KV caches need max_len %% 32 == 0 (got %d)", who, max_len);
  if (layout == HL_KV_TILED32 && stride % 8)
    return fail(HL_EINVAL, "%s: tiled KV caches need a batch stride multiple of 8", who);
  if (!aligned16(kc) || !aligned16(vc))
    return fail(HL_EINVAL, "%s: tiled and paged KV caches must be 16-byte aligned", who);
  if (layout == HL_KV_PAGED32) {
    if (!table) return fail(HL_EINVAL, "%s: paged KV caches need a block table", who);
    if (bps < max_len / 32)
      return fail(HL_EINVAL, "%s: blocks_per_seq %d < max_len/32 = %d", who, bps, max_len / 32);
  }
  return HL_OK;
}

// ---------------------------------------------------------------------------
// Decode attention
// ---------------------------------------------------------------------------
static int validate_decode(const hl_decode_args* a) {
  if (!a) return fail(HL_EINVAL, "decode: args is null");
  int rc = check_gqa(a->n_head, a->n_head_kv);
  if (rc) return rc;
  if ((rc = check_kv_dtype(a->kv_dtype, "decode kv_dtype"))) return rc;
  if (a->batch <= 0) return fail(HL_EINVAL, "decode: batch must be >= 1");
  if (a->head_dim != 64 && a->head_dim != 128)
    return fail(HL_EUNSUPPORTED, "decode: head_dim %d not built (64, 128)", a->head_dim);
  if (!a->q || !a->k_cache || !a->v_cache || !a->out) return fail(HL_EINVAL, "decode: null pointer");
  if (a->seq_len <= 0) return fail(HL_EINVAL, "decode: attention length must be >= 1");
  if (a->seq_len > a->max_len) return fail(HL_ECAPACITY, "KV cache full");
  if (a->num_splits < 0 || a->num_splits > 1024) return fail(HL_EINVAL, "decode: num_splits must be in [0, 1024]");
  if (!aligned16(a->q)) return fail(HL_EINVAL, "decode: q must be 16-byte aligned");
  const long long dense = (long long)a->n_head_kv * a->head_dim * a->max_len;
  if (a->cache_batch_stride != 0 && a->cache_batch_stride < dense)
    return fail(HL_EINVAL, "decode: cache_batch_stride smaller than one sequence's cache");
  return check_layout(a->kv_layout, a->kv_dtype, a->max_len, a->cache_batch_stride ? a->cache_batch_stride : dense,
                      a->k_cache, a->v_cache, a->block_table, a->blocks_per_seq, "decode");
}

size_t hl_attn_decode_workspace_bytes(const hl_decode_args* a) {
  if (validate_decode(a)) return 0;
  DecodePlan plan;
  decode_plan(a, &plan);
  return plan.ws_bytes;
}

int hl_attn_decode(const hl_decode_args* a, void* workspace, size_t ws_bytes, void* stream) {
  int rc = validate_decode(a);
  if (rc) return rc;
  DecodePlan plan;
  decode_plan(a, &plan);
  if (plan.ws_bytes > 0 && (!workspace || ws_bytes < plan.ws_bytes))
    return fail(HL_EINVAL, "decode: workspace of %zu bytes needed, %zu given", plan.ws_bytes, ws_bytes);
  if (plan.ws_bytes > 0 && ((uintptr_t)workspace & 3) != 0)
    return fail(HL_EINVAL, "decode: workspace must be 4-byte aligned");
  hipError_t e = decode_launch(a, &plan, workspace, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "decode launch");
}

int hl_attn_decode_workspace_init(void* workspace, size_t bytes, void* stream) {
  if (bytes == 0) return HL_OK;
  if (!workspace) return fail(HL_EINVAL, "decode workspace init: null pointer");
  hipError_t e = zero_fill_launch(workspace, bytes, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "workspace init launch");
}

// The gpuAttentionDecode call contract as batched args (B = 1, fp32 caches),
// validated and planned.
static int dropin_decode_plan(float* dst, const float* q, const float* k_cache, const float* v_cache, int n_head,
                              int n_head_kv, int head_dim, int cur_len, int cache_cols, hl_decode_args& a,
                              DecodePlan& plan) {
  memset(&a, 0, sizeof(a));
  a.batch = 1;
  a.n_head = n_head;
  a.n_head_kv = n_head_kv;
  a.head_dim = head_dim;
  a.kv_dtype = HL_F32;
  a.max_len = cache_cols;
  a.seq_len = cur_len;
  a.q = q;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.out = dst;
  int rc = validate_decode(&a);
  if (rc) return rc;
  decode_plan(&a, &plan);
  return HL_OK;
}

int hl_gpu_attention_decode(float* dst, const float* q, const float* k_cache, const float* v_cache,
                            int n_head, int n_head_kv, int head_dim, int cur_len, int cache_cols,
                            void* stream) {
  hl_decode_args a;
  DecodePlan plan;
  int rc = dropin_decode_plan(dst, q, k_cache, v_cache, n_head, n_head_kv, head_dim, cur_len, cache_cols, a, plan);
  if (rc) return rc;
  void* ws = nullptr;
  if (plan.ws_bytes > 0) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_mu);
    if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1);
    DevWs& w = g_ws[dev];
    if (w.bytes < plan.ws_bytes) {
      int rc = refuse_if_capturing(stream, "decode workspace");
      if (rc) return rc;
      if (w.ptr) {
        e = hipDeviceSynchronize();  // an earlier launch may still read it
        if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
        hipFree(w.ptr);
        w.ptr = nullptr;
        w.bytes = 0;
      }
      size_t bytes = plan.ws_bytes < (1u << 20) ? (1u << 20) : plan.ws_bytes;
      e = hipMalloc(&w.ptr, bytes);
      if (e != hipSuccess) return hip_fail(e, "hipMalloc(decode workspace)");
      e = hipMemset(w.ptr, 0, bytes);  // arrival counters start at zero
      if (e != hipSuccess) return hip_fail(e, "hipMemset(decode workspace)");
      w.bytes = bytes;
      w.zero_prefix = bytes;
    }
    // Bytes past the previous call's counters held its partials: a call with
    // a longer counter region clears the difference first.
    if (plan.counters_bytes > w.zero_prefix) {
      e = zero_fill_launch(w.ptr, plan.counters_bytes, as_stream(stream));
      if (e != hipSuccess) return hip_fail(e, "decode workspace clear");
    }
    w.zero_prefix = plan.counters_bytes;
    ws = w.ptr;
  }
  hipError_t e = decode_launch(&a, &plan, ws, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "decode launch");
}

// ---------------------------------------------------------------------------
// gpuAttentionDecode without any allocation: the split-K workspace is a
// fixed static device array instead of library-owned hipMalloc memory.
// ---------------------------------------------------------------------------
// One copy per device, held until the process ends.  Only its device address
// (hipGetSymbolAddress) is ever handed to a kernel or a fill: the array's
// name in host code is a host-side stand-in, not a device address.
constexpr size_t kNoAllocScratchBytes = (size_t)1 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
struct NoAllocDev {
  void* ptr = nullptr;      // device address of `scratch` on this device
  size_t zero_prefix = 0;   // leading bytes known to hold zero arrival counters
};
std::vector<NoAllocDev> g_noalloc;  // per device, guarded by g_mu
}  // namespace

int hl_gpu_attention_decode_noalloc(float* dst, const float* q, const float* k_cache, const float* v_cache,
                                    int n_head, int n_head_kv, int head_dim, int cur_len, int cache_cols,
                                    void* stream) {
  hl_decode_args a;
  DecodePlan plan;
  int rc = dropin_decode_plan(dst, q, k_cache, v_cache, n_head, n_head_kv, head_dim, cur_len, cache_cols, a, plan);
  if (rc) return rc;
  void* ws = nullptr;
  if (plan.ws_bytes > 0) {
    if (plan.ws_bytes > kNoAllocScratchBytes)
      return fail(HL_ECAPACITY, "decode_noalloc: this shape needs %zu bytes of split-K scratch; the static scratch holds %zu",
                  plan.ws_bytes, kNoAllocScratchBytes);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_mu);
    if ((int)g_noalloc.size() <= dev) g_noalloc.resize(dev + 1);
    NoAllocDev& d = g_noalloc[dev];
    if (!d.ptr) {  // first call on this device (which is current): its copy's address, then all zero
      void* ptr = nullptr;
      e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !ptr) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
      e = zero_fill_launch(ptr, kNoAllocScratchBytes, as_stream(stream));
      if (e != hipSuccess) return hip_fail(e, "decode_noalloc scratch clear");
      d.ptr = ptr;
      d.zero_prefix = kNoAllocScratchBytes;
    }
    // Every call leaves its arrival counters zero; bytes past the previous
    // call's counters held its partials, so a call with a longer counter
    // region clears the difference first (a fill kernel, no allocation).
    if (plan.counters_bytes > d.zero_prefix) {
      e = zero_fill_launch(d.ptr, plan.counters_bytes, as_stream(stream));
      if (e != hipSuccess) return hip_fail(e, "decode_noalloc counter clear");
    }
    d.zero_prefix = plan.counters_bytes;
    ws = d.ptr;
  }
  hipError_t e = decode_launch(&a, &plan, ws, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "decode launch");
}

// ---------------------------------------------------------------------------
// Decode-side fused qkNorm + RoPE + KV store
// ---------------------------------------------------------------------------
static int rope_store_op(const hl_rope_store_args* a, HeadVecOp& op) {
  if (!a) return fail(HL_EINVAL, "rope_store: args is null");
  int rc = check_gqa(a->n_head_q, a->n_head_kv);
  if (rc) return rc;
  if ((rc = check_kv_dtype(a->kv_dtype, "rope_store kv_dtype"))) return rc;
  if (a->batch <= 0 || a->head_dim <= 0 || a->head_dim > HL_MAX_HEAD_DIM || (a->head_dim & 1))
    return fail(HL_EINVAL, "rope_store: bad shape");
  if (!a->q || !a->k || !a->v || !a->k_cache || !a->v_cache) return fail(HL_EINVAL, "rope_store: null pointer");
  if (!a->positions && (a->pos < 0 || a->pos >= a->max_len)) return fail(HL_ECAPACITY, "KV cache full");
  const int rope_dim = a->rope_dim ? a->rope_dim : a->head_dim;
  if ((rc = check_rope(a->head_dim, rope_dim, a->rope_style))) return rc;
  const long long dense = (long long)a->n_head_kv * a->head_dim * a->max_len;
  if (a->cache_batch_stride != 0 && a->cache_batch_stride < dense)
    return fail(HL_EINVAL, "rope_store: cache_batch_stride smaller than one sequence's cache");
  if ((rc = check_layout(a->kv_layout, a->kv_dtype, a->max_len, a->cache_batch_stride ? a->cache_batch_stride : dense,
                         a->k_cache, a->v_cache, a->block_table, a->blocks_per_seq, "rope_store")))
    return rc;
  memset(&op, 0, sizeof(op));
  if ((rc = theta_for(a->use_installed_theta, rope_dim, a->rope_base, op.theta))) return rc;
  op.q = a->q;
  op.k = a->k;
  op.v = a->v;
  op.k_cache = a->k_cache;
  op.v_cache = a->v_cache;
  op.positions = a->positions;
  op.pos = a->pos;
  op.batch = a->batch;
  op.n_head_q = a->n_head_q;
  op.n_head_kv = a->n_head_kv;
  op.head_dim = a->head_dim;
  op.rope_dim = rope_dim;
  op.rope_style = a->rope_style;
  op.do_rope = 1;
  op.rope_q = 1;
  op.rope_k = 1;
  op.kv_dtype = a->kv_dtype;
  op.max_len = a->max_len;
  op.batch_stride = a->cache_batch_stride ? a->cache_batch_stride : dense;
  op.kv_layout = a->kv_layout;
  op.block_table = a->block_table;
  op.bps = a->blocks_per_seq;
  op.q_norm_w = a->q_norm_w;
  op.k_norm_w = a->k_norm_w;
  op.eps = a->eps;
  return HL_OK;
}

int hl_rope_store_decode(const hl_rope_store_args* a, void* stream) {
  HeadVecOp op;
  int rc = rope_store_op(a, op);
  if (rc) return rc;
  hipError_t e = headvec_launch(op, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "rope_store launch");
}

// ---------------------------------------------------------------------------
// Fused decode step: rope_store + attention in one launch (fp16/bf16 KV)
// ---------------------------------------------------------------------------
static int validate_step(const hl_rope_store_args* rs, const hl_decode_args* at, HeadVecOp& op) {
  int rc = rope_store_op(rs, op);
  if (rc) return rc;
  if ((rc = validate_decode(at))) return rc;
  if (rs->batch != at->batch || rs->n_head_q != at->n_head || rs->n_head_kv != at->n_head_kv ||
      rs->head_dim != at->head_dim || rs->kv_dtype != at->kv_dtype || rs->max_len != at->max_len ||
      rs->cache_batch_stride != at->cache_batch_stride || rs->q != at->q ||
      rs->k_cache != at->k_cache || rs->v_cache != at->v_cache || rs->kv_layout != at->kv_layout ||
      (at->kv_layout == HL_KV_PAGED32 &&
       (rs->block_table != at->block_table || rs->blocks_per_seq != at->blocks_per_seq)))
    return fail(HL_EINVAL, "decode_step: rope_store and decode args describe different tensors");
  if (at->seq_lens) return fail(HL_EINVAL, "decode_step: lengths come from the positions (seq_lens must be null)");
  if (!rs->positions && at->seq_len != rs->pos + 1)
    return fail(HL_EINVAL, "decode_step: seq_len must be pos + 1");
  return HL_OK;
}

static DecodeStep step_of(const HeadVecOp& op) {
  DecodeStep st;
  st.k = op.k;
  st.v = op.v;
  st.q_norm_w = op.q_norm_w;
  st.k_norm_w = op.k_norm_w;
  st.eps = op.eps;
  st.rope_dim = op.rope_dim;
  st.rope_style = op.rope_style;
  st.pos = op.pos;
  st.positions = op.positions;
  st.theta = op.theta;
  return st;
}

size_t hl_decode_step_workspace_bytes(const hl_rope_store_args* rs, const hl_decode_args* at) {
  HeadVecOp op;
  if (validate_step(rs, at, op)) return 0;
  DecodePlan plan;
  decode_plan(at, &plan, true);
  return plan.ws_bytes;
}

int hl_decode_step(const hl_rope_store_args* rs, const hl_decode_args* at, void* workspace,
                   size_t ws_bytes, void* stream) {
  HeadVecOp op;
  int rc = validate_step(rs, at, op);
  if (rc) return rc;
  DecodePlan plan;
  decode_plan(at, &plan, true);
  if (plan.ws_bytes > 0 && (!workspace || ws_bytes < plan.ws_bytes))
    return fail(HL_EINVAL, "decode_step: workspace of %zu bytes needed, %zu given", plan.ws_bytes, ws_bytes);
  if (plan.ws_bytes > 0 && ((uintptr_t)workspace & 3) != 0)
    return fail(HL_EINVAL, "decode_step: workspace must be 4-byte aligned");
  const hipStream_t s = as_stream(stream);
  const DecodeStep st = step_of(op);
  if (!plan.step) {  // fp32 KV: the stand-alone kernels, back to back
    hipError_t e = headvec_launch(op, s);
    if (e != hipSuccess) return hip_fail(e, "decode_step rope_store launch");
  }
  hipError_t e = decode_launch(at, &plan, workspace, s, &st);
  return e == hipSuccess ? HL_OK : hip_fail(e, "decode_step launch");
}

// ---------------------------------------------------------------------------
// Prefill
// ---------------------------------------------------------------------------
struct PrefillPlan {
  bool mfma;
  bool q_in_kernel;  // MFMA kernel builds Q from the raw activations (no qt)
  int t_pad;
  size_t off_q, off_k, off_v, off_tab, off_q32, off_k32, off_v32, off_range, bytes;
  size_t off_split, split_bytes;  // fp32: the K/V split images and their tile records
};

static int validate_prefill(const hl_prefill_args* a, PrefillPlan* pl) {
  if (!a) return fail(HL_EINVAL, "prefill: args is null");
  int rc = check_gqa(a->n_head, a->n_head_kv);
  if (rc) return rc;
  if ((rc = check_dtype(a->io_dtype, "prefill io_dtype"))) return rc;
  if (a->seq_len <= 0) return fail(HL_EINVAL, "prefill requires at least one token");
  if (a->head_dim != 64 && a->head_dim != 128)
    return fail(HL_EUNSUPPORTED, "prefill: head_dim %d not built (64, 128)", a->head_dim);
  if (!a->q || !a->k || !a->v || !a->out) return fail(HL_EINVAL, "prefill: null pointer");
  if (a->k_cache || a->v_cache) {
    if (!a->k_cache || !a->v_cache) return fail(HL_EINVAL, "prefill: give both caches or neither");
    if ((rc = check_kv_dtype(a->kv_dtype, "prefill kv_dtype"))) return rc;
    if (a->start_pos < 0) return fail(HL_EINVAL, "prefill: start_pos < 0");
    if ((long long)a->start_pos + a->seq_len > a->max_len)
      return fail(HL_ECAPACITY, "prefill exceeds KV cache capacity");
    if ((rc = check_layout(a->kv_layout, a->kv_dtype, a->max_len, 0, a->k_cache, a->v_cache,
                           a->block_table, a->max_len / 32, "prefill")))
      return rc;
  } else if (a->kv_layout != HL_KV_COLMAJOR && a->kv_layout != HL_KV_TILED32 &&
             a->kv_layout != HL_KV_PAGED32) {
    return fail(HL_EINVAL, "prefill: unknown kv_layout %d", a->kv_layout);
  }
  if (a->apply_rope) {
    const int rd = a->rope_dim ? a->rope_dim : a->head_dim;
    if ((rc = check_rope(a->head_dim, rd, a->rope_style))) return rc;
  }
  if ((rc = check_dtype(a->out_dtype, "prefill out_dtype"))) return rc;
  if (a->io_dtype == HL_F32 && a->out_dtype != HL_F32)
    return fail(HL_EUNSUPPORTED, "prefill: fp32 activations produce fp32 output");
  if (a->write_back_qk && a->io_dtype != HL_F32)
    return fail(HL_EUNSUPPORTED, "prefill: write_back_qk needs fp32 activations");
  const size_t D = a->head_dim, T = a->seq_len;
  pl->mfma = a->io_dtype != HL_F32;
  pl->off_split = pl->split_bytes = 0;
  const int rd = a->rope_dim ? a->rope_dim : a->head_dim;
  // The MFMA kernel applies RoPE to Q itself when every rotation pair lies in
  // one lane's registers: interleaved pairs, or half-split over all dims.
  pl->q_in_kernel = pl->mfma && (!a->apply_rope || a->rope_style == HL_ROPE_INTERLEAVED || rd == a->head_dim);
  if (pl->mfma) {
    pl->t_pad = prefill_mfma_tpad(a->seq_len);
    const size_t tp = pl->t_pad;
    pl->off_q = 0;
    pl->off_k = pl->off_q + (pl->q_in_kernel ? 0 : (size_t)a->n_head * tp * D * 2);
    pl->off_v = pl->off_k + (size_t)a->n_head_kv * tp * D * 2;
    pl->off_tab = pl->off_v + (size_t)a->n_head_kv * tp * D * 2;
    pl->bytes = pl->off_tab;
    if (a->apply_rope) pl->bytes += (size_t)T * (rd / 2) * 8;  // (cos, sin) table [rope_dim/2][T]
    // fp32 Q, K, V of the fallback pass (col-major, after qkNorm / RoPE)
    pl->off_q32 = (pl->bytes + 15) / 16 * 16;
    pl->off_k32 = pl->off_q32 + (size_t)a->n_head * D * T * 4;
    pl->off_v32 = pl->off_k32 + (size_t)a->n_head_kv * D * T * 4;
    pl->bytes = pl->off_v32 + (size_t)a->n_head_kv * D * T * 4;
    pl->off_range = (pl->bytes + 15) / 16 * 16;  // range record: mark, generation, staged generation, outcome
    pl->bytes = pl->off_range + 16;
  } else {
    pl->t_pad = a->seq_len;
    const bool pre = a->apply_rope || a->q_norm_w || a->k_norm_w;
    pl->off_q = 0;
    pl->off_k = (pre && !a->write_back_qk) ? (size_t)a->n_head * T * D * 4 : 0;
    pl->off_v = 0;
    pl->off_tab = 0;
    pl->off_q32 = pl->off_k32 = pl->off_v32 = 0;
    pl->off_range = 0;
    pl->bytes = (pre && !a->write_back_qk) ? pl->off_k + (size_t)a->n_head_kv * T * D * 4 : 0;
    pl->split_bytes = prefill_f32_split_bytes(a->n_head_kv, a->head_dim, a->seq_len);
    pl->off_split = (pl->bytes + 255) / 256 * 256;
    if (pl->split_bytes) pl->bytes = pl->off_split + pl->split_bytes;
  }
  return HL_OK;
}

}  // extern "C"

// Validation of the composed entry points' arguments (model.hip checks every
// layer's calls before launching anything).
int hl::check_decode_args(const hl_decode_args* a) { return validate_decode(a); }
int hl::check_step_args(const hl_rope_store_args* rs, const hl_decode_args* at) {
  HeadVecOp op;
  return validate_step(rs, at, op);
}
int hl::check_rope_store_args(const hl_rope_store_args* a) {
  HeadVecOp op;
  return rope_store_op(a, op);
}
int hl::check_prefill_args(const hl_prefill_args* a) {
  PrefillPlan pl;
  return validate_prefill(a, &pl);
}

extern "C" {

size_t hl_attn_prefill_workspace_bytes(const hl_prefill_args* a) {
  PrefillPlan pl;
  if (validate_prefill(a, &pl)) return 0;
  return pl.bytes;
}

// Fallback pass of an MFMA prefill, launched after every one: a Q*scale, K
// or V operand of magnitude >= 65520 has no fp16 form, and the prologue or
// the flash kernel then sets the range record's flag.  Two gated kernels
// follow; while the flag is clear each workgroup returns at once.  When it
// is set, the general prologue writes fp32 Q, K (after qkNorm / RoPE) and V
// from the original activations, and the fp32 flash kernel recomputes the
// whole output from them; its workgroup 0 advances the record's generation,
// which retires this call's mark.  The caches
// were already written with the exact values by the first prologue.
static int prefill_fallback(const hl_prefill_args* a, const PrefillPlan& pl, const PrologueOp& main_op,
                            float scale, char* ws, hipStream_t st) {
  unsigned* record = (unsigned*)(ws + pl.off_range);
  PrologueOp op = main_op;
  op.q = a->q;
  op.k = a->k;
  op.v = a->v;
  op.hv_first = 0;
  op.q_inplace = (float*)(ws + pl.off_q32);
  op.k_inplace = (float*)(ws + pl.off_k32);
  op.v_f32 = (float*)(ws + pl.off_v32);
  op.qt = op.kt = op.vt = nullptr;
  op.k_cache = op.v_cache = nullptr;
  op.block_table = nullptr;
  op.rope_tab_out = nullptr;
  op.range_word = nullptr;
  op.t_pad = a->seq_len;
  op.gate = record;
  hipError_t e = prologue_launch(op, st);
  if (e != hipSuccess) return hip_fail(e, "prefill fallback prologue launch");
  PrefillLaunch pf;
  memset(&pf, 0, sizeof(pf));
  pf.q = op.q_inplace;
  pf.k = op.k_inplace;
  pf.v = op.v_f32;
  pf.out = a->out;
  pf.out_dtype = a->out_dtype;
  pf.n_head = a->n_head;
  pf.n_head_kv = a->n_head_kv;
  pf.head_dim = a->head_dim;
  pf.seq_len = a->seq_len;
  pf.t_pad = a->seq_len;
  pf.scale_log2 = scale * kLog2e;
  pf.fallback_record = record;
  e = prefill_f32_launch(pf, st);
  return e == hipSuccess ? HL_OK : hip_fail(e, "prefill fallback launch");
}

int hl_attn_prefill(const hl_prefill_args* a, void* workspace, size_t ws_bytes, void* stream) {
  PrefillPlan pl;
  int rc = validate_prefill(a, &pl);
  if (rc) return rc;
  if (pl.bytes > 0 && (!workspace || ws_bytes < pl.bytes))
    return fail(HL_EINVAL, "prefill: workspace of %zu bytes needed, %zu given", pl.bytes, ws_bytes);
  if (pl.bytes > 0 && !aligned16(workspace)) return fail(HL_EINVAL, "prefill: workspace must be 16-byte aligned");
  const int rope_dim = a->rope_dim ? a->rope_dim : a->head_dim;
  PrologueOp op;
  memset(&op, 0, sizeof(op));
  if (a->apply_rope && (rc = theta_for(a->use_installed_theta, rope_dim, a->rope_base, op.theta)))
    return rc;
  const float scale = a->scale != 0.f ? a->scale : 1.0f / sqrtf((float)a->head_dim);
  char* ws = (char*)workspace;
  hipStream_t st = as_stream(stream);
  op.q = a->q;
  op.k = a->k;
  op.v = a->v;
  op.io_dtype = a->io_dtype;
  op.k_cache = a->k_cache;
  op.v_cache = a->v_cache;
  op.kv_dtype = a->kv_dtype;
  op.max_len = a->max_len;
  op.kv_layout = a->kv_layout;
  op.block_table = a->block_table;
  op.start_pos = a->start_pos;
  op.n_head = a->n_head;
  op.n_head_kv = a->n_head_kv;
  op.head_dim = a->head_dim;
  op.seq_len = a->seq_len;
  op.do_rope = a->apply_rope;
  op.rope_dim = rope_dim;
  op.rope_style = a->rope_style;
  op.q_norm_w = a->q_norm_w;
  op.k_norm_w = a->k_norm_w;
  op.eps = a->eps;
  op.t_pad = pl.t_pad;

  PrefillLaunch pf;
  memset(&pf, 0, sizeof(pf));
  pf.out = a->out;
  pf.out_dtype = a->out_dtype;
  pf.n_head = a->n_head;
  pf.n_head_kv = a->n_head_kv;
  pf.head_dim = a->head_dim;
  pf.seq_len = a->seq_len;
  pf.t_pad = pl.t_pad;
  hipError_t e;
  if (pl.mfma) {
    op.qt = pl.q_in_kernel ? nullptr : (uint16_t*)(ws + pl.off_q);
    op.kt = (uint16_t*)(ws + pl.off_k);
    op.vt = (uint16_t*)(ws + pl.off_v);
    op.qt_scale = scale * kLog2e;
    if (pl.q_in_kernel) {  // the prologue handles the k and v heads only
      op.q = nullptr;
      op.hv_first = a->n_head;
    }
    if (a->apply_rope) op.rope_tab_out = (float2*)(ws + pl.off_tab);  // written by the prologue
    unsigned* record = (unsigned*)(ws + pl.off_range);
    op.range_word = record;
    if ((e = prologue_launch(op, st)) != hipSuccess) return hip_fail(e, "prefill prologue launch");
    pf.qt = op.qt;
    pf.kt = op.kt;
    pf.vt = op.vt;
    pf.q_in = a->q;
    pf.io_dtype = a->io_dtype;
    pf.q_norm_w = a->q_norm_w;
    pf.eps = a->eps;
    pf.scale_log2 = scale * kLog2e;
    pf.do_rope = a->apply_rope;
    pf.rope_dim = rope_dim;
    pf.rope_style = a->rope_style;
    pf.rope_tab = op.rope_tab_out;
    pf.range_flag = record;
    if ((e = prefill_mfma_launch(pf, st)) != hipSuccess) return hip_fail(e, "prefill launch");
    return prefill_fallback(a, pl, op, scale, ws, st);
  }
  // fp32: normed/roped q,k either in place or in the workspace
  const bool pre = a->apply_rope || a->q_norm_w || a->k_norm_w;
  const float* qsrc = (const float*)a->q;
  const float* ksrc = (const float*)a->k;
  if (pre) {
    float* qd = a->write_back_qk ? (float*)a->q : (float*)(ws + pl.off_q);
    float* kd = a->write_back_qk ? (float*)a->k : (float*)(ws + pl.off_k);
    op.q_inplace = qd;
    op.k_inplace = kd;
    qsrc = qd;
    ksrc = kd;
  } else {
    op.q = nullptr;  // nothing to do for q; k only feeds the cache
    if (!a->k_cache) op.k = nullptr;
  }
  if (!a->k_cache) op.v = nullptr;
  if (pl.split_bytes) {
    // The prologue also writes the K/V split images the flash
    // kernel reads (so it always runs, over whole 64-token tiles).
    op.k = a->k;
    op.v = a->v;
    op.kv_img = ws + pl.off_split;
    op.kv_meta = (int*)(ws + pl.off_split + (size_t)a->n_head_kv * ((a->seq_len + 63) / 64) * split_img_bytes(a->head_dim));
    op.t_pad = (a->seq_len + 63) / 64 * 64;
    if (!op.q) op.hv_first = a->n_head;
    pf.kv_img = op.kv_img;
    pf.kv_meta = op.kv_meta;
  }
  if (op.q || op.k || op.v) {
    if ((e = prologue_launch(op, st)) != hipSuccess) return hip_fail(e, "prefill prologue launch");
  }
  pf.q = qsrc;
  pf.k = ksrc;
  pf.v = (const float*)a->v;
  pf.scale_log2 = scale * kLog2e;
  e = prefill_f32_launch(pf, st);
  return e == hipSuccess ? HL_OK : hip_fail(e, "prefill launch");
}

int hl_attn_prefill_fallback_ran(const hl_prefill_args* a, const void* workspace, int* ran, void* stream) {
  PrefillPlan pl;
  int rc = validate_prefill(a, &pl);
  if (rc) return rc;
  if (!ran) return fail(HL_EINVAL, "prefill fallback query: ran is null");
  *ran = 0;
  if (!pl.mfma) return HL_OK;
  if (!workspace) return fail(HL_EINVAL, "prefill fallback query: workspace is null");
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(as_stream(stream), &cs);
  if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
  if (cs != hipStreamCaptureStatusNone)
    return fail(HL_ECAPTURE, "prefill fallback query waits for the stream; it cannot run under stream capture");
  if ((e = hipStreamSynchronize(as_stream(stream))) != hipSuccess) return hip_fail(e, "prefill fallback query sync");
  unsigned w[4] = {0u, 0u, 0u, 0u};
  if ((e = hipMemcpy(w, (const char*)workspace + pl.off_range, sizeof(w), hipMemcpyDeviceToHost)) != hipSuccess)
    return hip_fail(e, "prefill fallback query read");
  *ran = w[3] != 0u ? 1 : 0;
  return HL_OK;
}

int hl_gpu_attention_prefill(float* dst, const float* q, const float* k, const float* v, int n_head,
                             int n_head_kv, int head_dim, int seq_len, void* stream) {
  hl_prefill_args a;
  memset(&a, 0, sizeof(a));
  a.n_head = n_head;
  a.n_head_kv = n_head_kv;
  a.head_dim = head_dim;
  a.seq_len = seq_len;
  a.io_dtype = HL_F32;
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = dst;
  PrefillPlan pl;
  int rc = validate_prefill(&a, &pl);
  if (rc) return rc;
  if (pl.bytes == 0) return hl_attn_prefill(&a, nullptr, 0, stream);
  // Library-owned workspace: the lock is held through the launch, so a
  // concurrent call that grows the buffer cannot free it under this one's
  // launches (it synchronises the device before freeing).
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_mu);
  if ((int)g_pws.size() <= dev) g_pws.resize(dev + 1);
  DevWs& w = g_pws[dev];
  if (w.bytes < pl.bytes) {
    if ((rc = refuse_if_capturing(stream, "prefill workspace"))) return rc;
    if (w.ptr) {
      e = hipDeviceSynchronize();  // an earlier launch may still read it
      if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
      hipFree(w.ptr);
      w.ptr = nullptr;
      w.bytes = 0;
    }
    e = hipMalloc(&w.ptr, pl.bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(prefill workspace)");
    w.bytes = pl.bytes;
  }
  return hl_attn_prefill(&a, w.ptr, w.bytes, stream);
}

static bool overlaps(const void* a, size_t abytes, const void* b, size_t bbytes) {
  const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
  return a0 < b0 + bbytes && b0 < a0 + abytes;
}

int hl_gpu_linear_col(float* dst, const float* x, const float* w, int w_cols, int w_rows,
                      int seq_len, void* stream) {
  if (!dst || !x || !w) return fail(HL_EINVAL, "linear_col: null pointer");
  if (w_cols <= 0 || w_rows <= 0 || seq_len <= 0)
    return fail(HL_EINVAL, "linear_col: bad shape (w_cols=%d, w_rows=%d, seq_len=%d)", w_cols,
                w_rows, seq_len);
  const size_t ybytes = (size_t)w_rows * seq_len * 4, xbytes = (size_t)w_cols * seq_len * 4;
  if (overlaps(dst, ybytes, x, xbytes) || overlaps(dst, ybytes, w, (size_t)w_rows * w_cols * 4))
    return fail(HL_EINVAL, "linear_col: dst overlaps x or w");
  hipError_t e = linear_col_launch(dst, x, w, w_cols, w_rows, seq_len, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "linear_col launch");
}

int hl_gpu_linear_col_quant(float* dst, const float* x, const void* w_quant, int w_cols, int w_rows,
                            int quant_type, void* stream) {
  if (!dst || !x || !w_quant) return fail(HL_EINVAL, "linear_col_quant: null pointer");
  const int qk = quant_block_elems(quant_type);
  if (qk == 0) return fail(HL_EUNSUPPORTED, "unsupported quant type for GPU GEMV: %d", quant_type);
  if (w_cols <= 0 || w_rows <= 0)
    return fail(HL_EINVAL, "linear_col_quant: bad shape (w_cols=%d, w_rows=%d)", w_cols, w_rows);
  if (quant_type != HL_GGML_F16 && w_cols % qk) {  // the rowSize* messages (quant.nim:27-73)
    const char* name = "";
    switch (quant_type) {
      case HL_GGML_Q5_0: name = "q5_0"; break;
      case HL_GGML_Q5_1: name = "q5_1"; break;
      case HL_GGML_Q8_0: name = "q8_0"; break;
      case HL_GGML_Q2_K: name = "q2_K"; break;
      case HL_GGML_Q3_K: name = "q3_K"; break;
      case HL_GGML_Q4_K: name = "q4_K"; break;
      case HL_GGML_Q5_K: name = "q5_K"; break;
      case HL_GGML_Q6_K: name = "q6_K"; break;
      case HL_GGML_IQ4_NL: name = "iq4_nl"; break;
    }
    return fail(HL_EINVAL, "%s row size must be multiple of %d", name, qk);
  }
  const size_t wbytes = (size_t)quant_row_bytes(quant_type, w_cols) * w_rows;
  if (overlaps(dst, (size_t)w_rows * 4, x, (size_t)w_cols * 4) || overlaps(dst, (size_t)w_rows * 4, w_quant, wbytes))
    return fail(HL_EINVAL, "linear_col_quant: dst overlaps x or w");
  hipError_t e = linear_quant_launch(dst, x, w_quant, w_cols, w_rows, quant_type, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "linear_col_quant launch");
}

int hl_gpu_rmsnorm_cols(float* dst, const float* x, const float* weight, int dim, int seq_len,
                        float eps, void* stream) {
  if (!dst || !x || !weight) return fail(HL_EINVAL, "rmsnorm_cols: null pointer");
  if (dim <= 0 || seq_len <= 0)
    return fail(HL_EINVAL, "rmsnorm_cols: bad shape (dim=%d, seq_len=%d)", dim, seq_len);
  if (!(eps >= 0.f)) return fail(HL_EINVAL, "rmsnorm_cols: eps must be >= 0");
  const size_t bytes = (size_t)dim * seq_len * 4;
  if (dst != x && overlaps(dst, bytes, x, bytes))
    return fail(HL_EINVAL, "rmsnorm_cols: dst partially overlaps x");
  hipError_t e = rmsnorm_cols_launch(dst, x, weight, dim, seq_len, eps, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "rmsnorm_cols launch");
}

int hl_gpu_residual_rmsnorm(float* norm_out, float* x, const float* residual, const float* weight,
                            int dim, float eps, void* stream) {
  if (!norm_out || !x || !residual || !weight)
    return fail(HL_EINVAL, "residual_rmsnorm: null pointer");
  if (dim <= 0) return fail(HL_EINVAL, "residual_rmsnorm: bad dim %d", dim);
  if (!(eps >= 0.f)) return fail(HL_EINVAL, "residual_rmsnorm: eps must be >= 0");
  if (overlaps(norm_out, (size_t)dim * 4, x, (size_t)dim * 4))
    return fail(HL_EINVAL, "residual_rmsnorm: norm_out overlaps x");
  hipError_t e = residual_rmsnorm_launch(norm_out, x, residual, weight, dim, eps, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "residual_rmsnorm launch");
}

// Library-owned argmax scratch of the current device (allocated and zeroed
// on the first call on that device).
static int argmax_scratch(unsigned int** out, void* stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_mu);
  if ((int)g_argmax_ws.size() <= dev) g_argmax_ws.resize(dev + 1, nullptr);
  if (!g_argmax_ws[dev]) {
    void* p = nullptr;
    int rc = refuse_if_capturing(stream, "argmax scratch");
    if (rc) return rc;
    e = hipMalloc(&p, kArgmaxScratchBytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(argmax scratch)");
    e = hipMemset(p, 0, kArgmaxScratchBytes);
    if (e != hipSuccess) return hip_fail(e, "hipMemset(argmax scratch)");
    g_argmax_ws[dev] = p;
  }
  *out = (unsigned int*)g_argmax_ws[dev];
  return HL_OK;
}

int hl_argmax_async(const float* logits, int n_vocab, int32_t* result_dev, void* stream) {
  if (!logits || !result_dev) return fail(HL_EINVAL, "argmax: null pointer");
  if (n_vocab < 0) return fail(HL_EINVAL, "argmax: n_vocab %d < 0", n_vocab);
  unsigned int* scratch = nullptr;
  int rc = argmax_scratch(&scratch, stream);
  if (rc) return rc;
  hipError_t e = argmax_launch(logits, n_vocab, scratch, result_dev, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "argmax launch");
}

int hl_gpu_argmax(const float* logits, int n_vocab, int32_t* result, void* stream) {
  if (!logits || !result) return fail(HL_EINVAL, "argmax: null pointer");
  if (n_vocab < 0) return fail(HL_EINVAL, "argmax: n_vocab %d < 0", n_vocab);
  unsigned int* scratch = nullptr;
  int rc = argmax_scratch(&scratch, stream);
  if (rc) return rc;
  int* slot = (int*)((char*)scratch + kArgmaxScratchBytes - 8);
  hipError_t e = argmax_launch(logits, n_vocab, scratch, slot, as_stream(stream));
  if (e != hipSuccess) return hip_fail(e, "argmax launch");
  e = hipMemcpyAsync(result, slot, sizeof(int32_t), hipMemcpyDeviceToHost, as_stream(stream));
  if (e != hipSuccess) return hip_fail(e, "argmax copy");
  e = hipStreamSynchronize(as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "argmax sync");
}

int hl_gpu_embedding(float* dst, const float* weight, const int32_t* token_ids, int n_emb,
                     int n_tokens, int n_vocab, void* stream) {
  if (!dst || !weight || !token_ids) return fail(HL_EINVAL, "embedding: null pointer");
  if (n_emb <= 0 || n_tokens <= 0 || n_vocab <= 0)
    return fail(HL_EINVAL, "embedding: bad shape (n_emb=%d, n_tokens=%d, n_vocab=%d)", n_emb,
                n_tokens, n_vocab);
  hipError_t e = embedding_launch(dst, weight, token_ids, n_emb, n_tokens, n_vocab, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "embedding launch");
}

int hl_kv_cache_to_f32(float* dst, const void* cache, int kv_dtype, int rows, int max_len, int col0,
                       int ncols, void* stream) {
  if (!dst || !cache) return fail(HL_EINVAL, "cache_to_f32: null pointer");
  int rc = check_kv_dtype(kv_dtype, "cache_to_f32");
  if (rc) return rc;
  if (rows <= 0 || ncols <= 0 || col0 < 0 || col0 + ncols > max_len)
    return fail(HL_EINVAL, "cache_to_f32: bad range");
  hipError_t e = cache_to_f32_launch(dst, cache, kv_dtype, rows, max_len, col0, ncols, as_stream(stream));
  return e == hipSuccess ? HL_OK : hip_fail(e, "cache_to_f32 launch");
}

}  // extern "C"
