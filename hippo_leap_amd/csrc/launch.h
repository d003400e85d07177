// Internal host-side launchers shared between the kernel translation units
// and the C-ABI layer (api.hip).  Validation happens in api.hip; these assume
// arguments already checked.
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace hl {

// ---- decode attention (decode.hip) ----------------------------------------
struct DecodePlan {
  int head_chunk, n_chunks, num_splits, split_len;
  bool vec;             // 16-byte cache loads (fp16/bf16, aligned rows)
  bool pipe;            // prefetching kernel (several tiles per wave)
  bool step;            // fused decode step (qkNorm + RoPE + cache write inside)
  size_t counters_bytes;  // arrival counters at the workspace start, partials after
  size_t ws_bytes;
};
// The new token's inputs of a fused decode step (fp16/bf16 KV): a->q is then
// the raw q activation, and the kernel ropes q and k, writes k and v into
// cache column pos (positions[b] if given) and attends over pos + 1 columns.
struct DecodeStep {
  const float* k;
  const float* v;
  const float* q_norm_w;
  const float* k_norm_w;
  float eps;
  int rope_dim, rope_style, pos;
  const int* positions;
  ThetaTable theta;
};
void decode_plan(const hl_decode_args* a, DecodePlan* plan, bool step = false);
hipError_t decode_launch(const hl_decode_args* a, const DecodePlan* plan, void* ws,
                         hipStream_t stream, const DecodeStep* step = nullptr);
hipError_t zero_fill_launch(void* ws, size_t bytes, hipStream_t stream);

// ---- per-token head-vector ops (rope_store.hip) ---------------------------
// One launch over B sequences x (Hq + 2*Hkv) head vectors of the new token:
// optional RMSNorm, optional RoPE at the sequence's position, optional store
// of k / v into the cache column.
struct HeadVecOp {
  float* q;            // [B][Hq*D] or null
  float* k;            // [B][Hkv*D] or null
  const float* v;      // [B][Hkv*D] or null
  void* k_cache;       // null: no store
  void* v_cache;
  const int* positions;
  int pos;
  int batch, n_head_q, n_head_kv, head_dim, rope_dim, rope_style, do_rope, kv_dtype, max_len;
  int kv_layout;       // HL_KV_COLMAJOR | HL_KV_TILED32 | HL_KV_PAGED32
  const int* block_table;  // paged: [B][bps]
  int bps;
  long long batch_stride;
  const float* q_norm_w;
  const float* k_norm_w;
  float eps;
  int rope_q, rope_k;  // which tensors get RoPE
  ThetaTable theta;
};
hipError_t headvec_launch(const HeadVecOp& op, hipStream_t stream);

// ---- column-major prologue (rope_store.hip) --------------------------------
// Works on col-major [H*D, T] activations, one (head, 64-column tile) per
// workgroup, for the Q heads, K heads and V heads of a prefill:
//   Q: norm?, RoPE?, then write back in place (fp32) and/or to the MFMA
//      layout qt[Hq][T][D] (fp16, pre-scaled by scale*log2 e)
//   K: norm?, RoPE?, write back / kt[Hkv][T][D] fp16 / cache column
//   V: vt[Hkv][D][T] fp16 and/or cache column
struct PrologueOp {
  const void* q;
  const void* k;
  const void* v;
  int io_dtype;
  float* q_inplace;   // fp32 write-back targets (may alias q/k) or null
  float* k_inplace;
  float* v_f32;       // fp32 copy of v (col-major [Hkv*D, T]) or null
  uint16_t* qt;       // MFMA layouts (fp16 bits) or null
  uint16_t* kt;
  uint16_t* vt;
  void* k_cache;
  void* v_cache;
  int kv_dtype, max_len, start_pos;
  int kv_layout;      // of the caches: HL_KV_COLMAJOR | HL_KV_TILED32 | HL_KV_PAGED32
  const int* block_table;  // paged: this sequence's pages
  int n_head, n_head_kv, head_dim, seq_len;
  int do_rope, rope_dim, rope_style;
  const float* q_norm_w;
  const float* k_norm_w;
  float eps;
  float qt_scale;     // multiplier folded into qt
  int t_pad;          // row count of qt/kt/vt (seq_len rounded up); pad rows zeroed
  int hv_first;       // first head vector processed (n_head: k and v heads only)
  int hpg;            // head vectors per workgroup (set by prologue_launch)
  int n_tiles, n_hgrps;  // work items: 32-token tiles x head groups (set by prologue_launch)
  ThetaTable theta;
  float2* rope_tab_out;  // optional: receives the (cos, sin) table [rope_dim/2][seq_len] of
                         // positions start_pos + t (rope_dim/2 <= 64)
  // Range record of the fp16 operands (qt / kt / vt): see range_flag_set in
  // common.h.  A thread whose operand value has magnitude >= kF16Inf marks
  // it.  Null: not recorded.
  unsigned* range_word;
  // Fallback pass: non-null -> every workgroup returns at once unless
  // gate[0] (the overflow flag) is set.
  unsigned* gate;
  // fp32 prefill: the K and V split images and tile records
  // of the flash kernel (PrefillLaunch::kv_img / kv_meta), or null.
  // t_pad must then be seq_len rounded up to 64.
  char* kv_img;
  int* kv_meta;
};
hipError_t prologue_launch(const PrologueOp& op, hipStream_t stream);

// Plain column copy with dtype conversion: cache[r*cache_cols + start + c] =
// src[r*src_cols + c] (two tensors when src2 != null).
hipError_t store_cols_launch(void* cache, const float* src, void* cache2, const float* src2,
                             int rows, int src_cols, int cache_cols, int start_pos, int kv_dtype,
                             hipStream_t stream);

hipError_t cache_to_f32_launch(float* dst, const void* cache, int kv_dtype, int rows, int max_len,
                               int col0, int ncols, hipStream_t stream);

// ---- prefill attention (prefill.hip) --------------------------------------
struct PrefillLaunch {
  // fp32 path: col-major q/k/v/out [H*D, T]
  const float* q;
  const float* k;
  const float* v;
  // MFMA path: qt [Hq][Tp][D], kt [Hkv][Tp][D], vt [Hkv][D][Tp] (fp16 bits)
  const uint16_t* qt;  // null: the MFMA kernel builds Q from q_in itself
  const uint16_t* kt;
  const uint16_t* vt;
  void* out;
  int out_dtype;
  int n_head, n_head_kv, head_dim, seq_len, t_pad;
  float scale_log2;   // fp32 path; MFMA path: folded into qt, or applied to q_in
  // MFMA path with qt == null: raw col-major q [Hq*D, T] in io_dtype, with
  // optional qkNorm and RoPE (full-dimension half-split, or interleaved)
  const void* q_in;
  int io_dtype;
  const float* q_norm_w;
  float eps;
  int do_rope, rope_dim, rope_style;
  const float2* rope_tab;  // [rope_dim/2][seq_len]
  // Q built in the kernel: a lane whose Q operand value (q * scale, after
  // qkNorm / RoPE) has magnitude >= kF16Inf sets *range_flag.
  unsigned* range_flag;
  // fp32 kernel as the fallback pass of an MFMA prefill: the range record.
  // Workgroups return at once unless the call's overflow mark is set;
  // workgroup 0 advances the record's generation (common.h).
  unsigned* fallback_record;
  // fp32 path (not the fallback pass): the K/V split images
  // the prologue writes (PrologueOp::kv_img) and the flash kernel reads,
  // prefill_f32_split_bytes in all: [Hkv][ceil(T/64)] images of 32 KB, then
  // a record of 8 ints per image (kSplitRec*).
  void* kv_img;
  int* kv_meta;
};
hipError_t prefill_f32_launch(const PrefillLaunch& p, hipStream_t stream);
size_t prefill_f32_split_bytes(int n_head_kv, int head_dim, int seq_len);
hipError_t prefill_mfma_launch(const PrefillLaunch& p, hipStream_t stream);
int prefill_mfma_tpad(int seq_len);

// ---- fp32 linear layer (linear.hip) ----------------------------------------
// Y[M, T] = W[M, K] . X[K, T]: GEMV for T == 1, fp32-MFMA GEMM otherwise.
struct LinearPlan {
  bool gemv;
  bool vec;      // 16-byte loads (K % 4 == 0, T % 4 == 0 for the GEMM, aligned w, x)
  int wpr;       // GEMV: waves per row (1, or 4 when M is small)
  int tile;      // GEMM: output tile edge (64 or 128)
  int grid_x, grid_y;
};
LinearPlan linear_plan(int M, int K, int T, const float* w, const float* x);
hipError_t linear_col_launch(float* y, const float* x, const float* w, int K, int M, int T,
                             hipStream_t stream);

// ---- quantized decode GEMV (linear_quant.hip) ------------------------------
int cu_count();                          // CUs of the current device (cached)
int quant_block_elems(int qtype);        // 0: type not built

// ---- argument validation of the C-ABI entry points (api.hip) --------------
// HL_OK or the entry point's own error code and message.
int check_decode_args(const hl_decode_args* a);
int check_step_args(const hl_rope_store_args* rs, const hl_decode_args* at);
int check_rope_store_args(const hl_rope_store_args* a);
int check_prefill_args(const hl_prefill_args* a);
long long quant_row_bytes(int qtype, int K);
hipError_t linear_quant_launch(float* y, const float* x, const void* w, int K, int M, int qtype,
                               hipStream_t stream);

// ---- RMSNorm of the hidden state (norm.hip) --------------------------------
hipError_t rmsnorm_cols_launch(float* out, const float* x, const float* w, int dim, int seq,
                               float eps, hipStream_t stream);
hipError_t residual_rmsnorm_launch(float* out, float* x, const float* res, const float* w, int dim,
                                   float eps, hipStream_t stream);
// x_dst = x_in + res; out = rmsnorm(x_dst) * w (out may be x_in).
hipError_t residual_rmsnorm_from_launch(float* out, float* x_dst, const float* x_in, const float* res,
                                        const float* w, int dim, float eps, hipStream_t stream);

// ---- decode-step ends: argmax and embedding (tokens.hip) -------------------
constexpr int kArgmaxMaxGroups = 256;
// Scratch: an 8-byte arrival counter (zero between calls), one 8-byte key
// per workgroup, then the 4-byte result slot used by the host-result entry.
constexpr size_t kArgmaxScratchBytes = 8 + 8 * kArgmaxMaxGroups + 8;
int argmax_grid(int n);
hipError_t argmax_launch(const float* x, int n, unsigned int* scratch, int* result,
                         hipStream_t stream);
hipError_t embedding_launch(float* out, const float* w, const int* tok, int n_emb, int n_tok,
                            int n_vocab, hipStream_t stream);

bool linear_quant_pair_launch(int pair, float* y, float* y2, const float* x, const void* wa,
                              const void* wb, int K, int M, int qtype, hipStream_t stream);
// Q, K and V projections of one x in one launch (false: run them apart).
bool linear_quant_qkv_launch(float* yq, float* yk, float* yv, const float* x, const void* wq, const void* wk,
                             const void* wv, int K, int Mq, int Mkv, int qtype, hipStream_t stream);
// xsum = x + res, then the fused gate/up/SiLU of rmsnorm(xsum) * nrm in one
// launch (Q4_K on the matrix cores, K <= 8192); false when not applicable.
bool linear_quant_gate_up_norm_launch(float* y, float* xsum, const float* x, const float* res, const float* nrm,
                                      float eps, const void* wg, const void* wu, int K, int M, int qtype,
                                      hipStream_t stream);

// Sets the thread's hl_last_error() message (printf format); returns code.
int set_error(int code, const char* fmt, ...);

}  // namespace hl
