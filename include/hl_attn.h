/*
 * hl_attn.h — C ABI of the MI355X (gfx950) attention stage for HippoLeap.
 *
 * The library (libhl_attn.so) replaces the attention sub-sequence of the
 * reference's naive backend: per-head RMSNorm (qkNorm) -> RoPE -> KV-cache
 * store -> attention.  Reference files are cited relative to the
 * monofuel/hippo_leap repository root.
 *
 * Conventions shared by every entry point
 *  - Plain pointers and sizes only; `stream` is a hipStream_t passed as void*
 *    (NULL = the null stream).  All work is enqueued asynchronously on that
 *    stream; nothing synchronises, nothing allocates device memory except
 *    the library-owned scratch of two reference-signature drop-ins
 *    (hl_gpu_attention_decode's split-K workspace, grown when a call needs
 *    more; hl_gpu_argmax / hl_argmax_async's 2 KB, on the first call on a
 *    device).  Those allocations synchronise the device; while `stream` is
 *    being captured into a HIP graph they are refused with HL_ECAPTURE
 *    instead (make one call of the largest shape before capturing).
 *  - The caller owns every device buffer (naive.nim:171-182).
 *  - Return value: HL_OK (0) or a negative HL_E* code.  hl_last_error()
 *    returns a thread-local message for the last failing call, mirroring the
 *    reference's `raise newException(ValueError, msg)` (naive.nim:3969-3976,
 *    4594-4599).
 *  - Layouts follow the reference ("ggml column-major"): a `[R, C]` tensor
 *    stores element (r, c) at r*C + c, so the column index (token / cache
 *    position) is fastest.
 *      decode vectors q/k/v/out : [B][H*D]           (naive.nim:4697-4717)
 *      prefill activations      : [H*D, T]           (naive.nim:4064-4078)
 *      KV cache (one layer)     : [Hkv*D, max_len]   (naive.nim:3565-3567)
 *    For B > 1, sequence b's cache starts cache_batch_stride elements after
 *    sequence b-1's (0 = dense: Hkv*D*max_len).
 */
#ifndef HL_ATTN_H
#define HL_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
enum {
  HL_OK = 0,
  HL_EINVAL = -1,        /* bad shape / pointer / GQA divisibility          */
  HL_ECAPACITY = -2,     /* KV cache full, prefill longer than max_len      */
  HL_EUNSUPPORTED = -3,  /* dtype / head_dim combination not built          */
  HL_EHIP = -4,          /* HIP runtime error (launch, device query)         */
  HL_ECAPTURE = -5       /* would allocate while the stream is being captured */
};

/* ---- element types of activations and KV cache ------------------------- */
/* HL_FP8: OCP fp8 e4m3 ("e4m3fn": bias 7, no infinities, max 448), KV caches
 * only and only in the HL_KV_TILED32 layout.  Writes round to nearest even
 * and saturate to +-448 (infinities too; NaN stays NaN); reads are exact.
 * Extends the reference, which keeps fp32 caches.                          */
enum { HL_F32 = 0, HL_F16 = 1, HL_BF16 = 2, HL_FP8 = 3 };

/* ---- RoPE pairing ------------------------------------------------------- */
enum {
  HL_ROPE_HALF_SPLIT = 0,  /* pairs (i, i+rope_dim/2): every GPU kernel of the
                              reference (naive.nim:3020-3030, 3066-3073)     */
  HL_ROPE_INTERLEAVED = 1  /* pairs (2i, 2i+1): tensor.nim:141-166           */
};

#define HL_MAX_HEAD_DIM 256
#define HL_MAX_ROPE_DIM 256

/* ------------------------------------------------------------------------ */
/* Library state and diagnostics                                             */
/* ------------------------------------------------------------------------ */

/* Message of the last failing call on this thread ("" if none). */
const char* hl_last_error(void);

/* ABI version: bumped when a struct below changes. */
int hl_abi_version(void);

typedef struct hl_device_info {
  int device;
  int cu_count;
  int clock_khz;             /* peak engine clock                         */
  int mem_clock_khz;
  int l2_bytes;
  size_t hbm_bytes;
  double hbm_peak_gbs;       /* published MI355X HBM3E peak (8000 GB/s)   */
  double bf16_dense_tflops;  /* CUs x clk x 4096 flop/clk/CU (dense MFMA) */
  double fp32_tflops;        /* published vector fp32 peak                */
  char arch[64];             /* e.g. "gfx950:sramecc+:xnack-"             */
} hl_device_info;

/* Fills *info for the current HIP device.  Replaces nothing in the
 * reference (which has no roofline reporting); used by the benchmark.     */
int hl_device_info_get(hl_device_info* info);

/* Measurement probe, no counterpart in the reference: one launch of
 * `blocks` workgroups (0 -> 1024) that streams `bytes` (a multiple of 16,
 * 16-byte aligned) from device memory with 16-byte loads and computes
 * nothing else (`sink`: a device word it practically never writes).  It is
 * the floor a kernel reading that many bytes once reaches on this part,
 * timed beside the decode kernels at their byte counts.                    */
int hl_probe_stream_read(const void* buf, size_t bytes, int blocks, unsigned* sink, void* stream);
/* The same probe with `inflight` (4, 8 or 16) 16-byte loads per thread per
 * iteration, and with contiguous != 0 each workgroup streaming its own
 * contiguous chunk instead of a grid-stride sweep.                        */
int hl_probe_stream_read_ex(const void* buf, size_t bytes, int blocks, int inflight, int contiguous,
                            unsigned* sink, void* stream);

/* Host-side RoPE theta table: theta[i] = powf(1/base, 2i/rope_dim) for
 * i < rope_dim/2, computed in fp32 exactly as naive.nim:3850-3861.       */
int hl_rope_theta_table(float* theta_out, int rope_dim, float rope_base);

/* Installs the process-wide theta table used by the entry points that, in
 * the reference, read modelPtrs.ropeTheta (gpuRopeQKDecode,
 * gpuRopeAtPosTheta, gpuFusedRopeStoreKV).  Mirrors the table build inside
 * ensureModelGpuPtrs / loadModelBackend (naive.nim:3850-3861, 3956-3958).
 * The table travels to the GPU as a kernel argument: no device memory.   */
int hl_set_rope_theta(int rope_dim, float rope_base);

/* ------------------------------------------------------------------------ */
/* Drop-ins with the reference's exact call contract (fp32, one sequence).   */
/* Argument order and meaning follow the Nim procs cited on each line.       */
/* ------------------------------------------------------------------------ */

/* gpuQkNorm (naive.nim:2918-2926): per-head RMSNorm of x[nHead*headDim] in
 * place, x * (1/sqrtf(sum(x^2)/headDim + eps)) * w[d].                     */
int hl_gpu_qk_norm(float* x, const float* weight, int n_head, int head_dim,
                   float eps, void* stream);

/* gpuQkNormPrefill (naive.nim:2962-2971): same on col-major [nHead*headDim,
 * seqLen], one normalisation per (head, column).                          */
int hl_gpu_qk_norm_prefill(float* x, const float* weight, int n_head,
                           int head_dim, int seq_len, float eps, void* stream);

/* gpuRopeAtPos (naive.nim:3088-3101): half-split RoPE in place.  seq_len==1:
 * x is [nHead*headDim] at position `pos`; seq_len>1: x is col-major
 * [nHead*headDim, seqLen] and column p is rotated at position p (the
 * reference ignores `pos` there, naive.nim:3036-3037).  Theta is
 * powf(1/ropeBase, 2i/ropeDim) evaluated on the host.                      */
int hl_gpu_rope_at_pos(float* x, int n_head, int head_dim, int rope_dim,
                       float rope_base, int pos, int seq_len, void* stream);

/* gpuRopeAtPosTheta (naive.nim:3133-3144): as above with the installed theta
 * table; for seq_len>1 column p is rotated at position pos+p.              */
int hl_gpu_rope_at_pos_theta(float* x, int n_head, int head_dim, int rope_dim,
                             int pos, int seq_len, void* stream);

/* gpuRopeQKDecode (naive.nim:3075-3086): RoPE of q[nHeadQ*headDim] and
 * k[nHeadK*headDim] at `pos` in one launch with the installed theta table
 * (the reference ignores ropeBase; so does this entry point when a table is
 * installed, otherwise the table is built from rope_base).               */
int hl_gpu_rope_qk_decode(float* q, float* k, int n_head_q, int n_head_k,
                          int head_dim, int rope_dim, float rope_base, int pos,
                          void* stream);

/* gpuFusedRopeStoreKV (naive.nim:3203-3223): RoPE q,k at `pos` in place,
 * then write rotated k and v into column `pos` of the fp32 caches
 * [kvDim, cacheCols]; dims >= ropeDim of k are copied unrotated.          */
int hl_gpu_fused_rope_store_kv(float* q, float* k, const float* v,
                               float* k_cache, float* v_cache, int n_head_q,
                               int n_head_k, int head_dim, int rope_dim,
                               int kv_dim, int cache_cols, int pos,
                               void* stream);

/* gpuStoreKV (naive.nim:3241-3253): cache[r*cacheCols + startPos + c] =
 * src[r*srcCols + c] for r < rows, c < srcCols.                          */
int hl_gpu_store_kv(float* cache, const float* src, int rows, int src_cols,
                    int cache_cols, int start_pos, void* stream);

/* gpuStoreKVPair (naive.nim:3273-3285): gpuStoreKV of K and V in one launch. */
int hl_gpu_store_kv_pair(float* k_cache, const float* k_src, float* v_cache,
                         const float* v_src, int rows, int src_cols,
                         int cache_cols, int start_pos, void* stream);

/* gpuAttentionDecode (naive.nim:3369-3383): dst[nHead*headDim] =
 * softmax(q_h . K^T / sqrt(headDim)) . V over cache columns [0, curLen) of
 * the fp32 caches [nHeadKv*headDim, cacheCols], kv head = h / (nHead /
 * nHeadKv).  Split-K over the context with a library-owned workspace, one
 * per device and shared by every stream: like the reference, which runs
 * the whole backend on one stream (naive.nim:241-244), callers on one
 * device must not overlap calls on different streams.  A call that needs a
 * larger workspace than any before it on the device allocates it
 * (synchronising the device); under stream capture it returns HL_ECAPTURE. */
int hl_gpu_attention_decode(float* dst, const float* q, const float* k_cache,
                            const float* v_cache, int n_head, int n_head_kv,
                            int head_dim, int cur_len, int cache_cols,
                            void* stream);

/* hl_gpu_attention_decode without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results as
 * hl_gpu_attention_decode; its split-K workspace is a static 1 MiB device
 * array of the library (one copy per device, held until the process ends)
 * instead of hipMalloc memory, so it never allocates, frees or synchronises.
 * A shape whose split-K partials (nHead * splits * (headDim + 2) * 4 bytes,
 * plus 256) exceed 1 MiB returns HL_ECAPACITY before launching anything;
 * that takes hundreds of query heads (32 heads need at most ~0.3 MiB).  Every
 * call on a device shares that device's array: calls that overlap in time
 * on one device (e.g. on two streams) race.  The first call on a device
 * zero-fills the array with a kernel on `stream`.                       */
int hl_gpu_attention_decode_noalloc(float* dst, const float* q, const float* k_cache,
                                    const float* v_cache, int n_head, int n_head_kv,
                                    int head_dim, int cur_len, int cache_cols,
                                    void* stream);

/* gpuAttentionPrefill (naive.nim:3450-3464): causal attention over the
 * col-major fp32 projections q[nHead*headDim, seqLen], k/v[nHeadKv*headDim,
 * seqLen]; dst is col-major [nHead*headDim, seqLen].  No 4096-token cap.
 * It uses a library-owned workspace per device (the K/V
 * split images, hipMalloc'd when a call needs more than the last one and
 * kept; growing it waits for the device and is refused under capture).  */
int hl_gpu_attention_prefill(float* dst, const float* q, const float* k,
                             const float* v, int n_head, int n_head_kv,
                             int head_dim, int seq_len, void* stream);

/* gpuLinearCol (naive.nim:3519-3547), the Q/K/V and O projections around
 * attention: dst[wRows, seqLen] = w[wRows, wCols] . x[wCols, seqLen], all
 * fp32; w row-major (wCols fastest), x and dst with seqLen fastest.
 * seq_len == 1 is the decode GEMV, seq_len > 1 the prefill GEMM.  dst must
 * not overlap x or w (HL_EINVAL: the outputs would race with the reads).
 * Unlike the reference's decode kernel there is no width cap
 * (HippoMaxDecodeCols = 18432, naive.nim:20, 3530-3533).                 */
int hl_gpu_linear_col(float* dst, const float* x, const float* w, int w_cols,
                      int w_rows, int seq_len, void* stream);

/* GGUF weight types of hl_gpu_linear_col_quant (ggml's type ids, as the
 * reference's GgmlType* constants, model.nim:11-21).                        */
enum {
  HL_GGML_F16 = 1, HL_GGML_Q5_0 = 6, HL_GGML_Q5_1 = 7, HL_GGML_Q8_0 = 8,
  HL_GGML_Q2_K = 10, HL_GGML_Q3_K = 11, HL_GGML_Q4_K = 12, HL_GGML_Q5_K = 13,
  HL_GGML_Q6_K = 14, HL_GGML_IQ4_NL = 20
};

/* gpuLinearColQuant (naive.nim:1580-1592): dst[wRows] = dequant(w)[wRows,
 * wCols] . x[wCols] for one token (the reference's quantized GEMVs are
 * decode-only), with w the GGUF rows of quant_type, every type the
 * reference dispatches: F16, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K,
 * IQ4_NL (dequantisation as quant.nim:132-441; Q5_K as the reference's GPU
 * kernel, naive.nim:1267-1323).  wCols must be a multiple of the block (32;
 * 256 for the K-quants; any for F16): HL_EINVAL with the reference's
 * row-size message otherwise.  Other types: HL_EUNSUPPORTED ("unsupported
 * quant type for GPU GEMV: <type>").  dst must not overlap x or w.        */
int hl_gpu_linear_col_quant(float* dst, const float* x, const void* w_quant,
                            int w_cols, int w_rows, int quant_type,
                            void* stream);

/* gpuRmsnormCols (naive.nim:2834-2843): dst[r, t] = x[r, t] *
 * (1/sqrtf(sum_r x[r, t]^2 / dim + eps)) * weight[r] over the col-major
 * fp32 [dim, seqLen] (the norm in front of the Q/K/V projections and the
 * final norm before the logits).  dst may equal x.                        */
int hl_gpu_rmsnorm_cols(float* dst, const float* x, const float* weight,
                        int dim, int seq_len, float eps, void* stream);

/* gpuResidualRmsnorm (naive.nim:2874-2882): x[r] += residual[r] in place,
 * then norm_out[r] = x[r] * (1/sqrtf(sum x^2 / dim + eps)) * weight[r]
 * (one vector, the end of a decode layer).  norm_out must not overlap x.  */
int hl_gpu_residual_rmsnorm(float* norm_out, float* x, const float* residual,
                            const float* weight, int dim, float eps,
                            void* stream);

/* gpuArgmax (naive.nim:2105-2127): index of the greedy token over
 * logits[nVocab] (fp32, device), written to *result (host) after the stream
 * has finished, as the reference returns it after gpuStreamSync.  Same
 * result as the reference's two-pass kernel (naive.nim:1922-2103) on every
 * input, ties included: among equal maxima at i = 65536r + 256b + t the
 * smallest (bitrev8(b), bitrev8(t), r) wins, which is where the reference's
 * 256x256-thread reduction tree puts them; NaN and values <= -3.4e38 are
 * never chosen; -1 if nothing is.  Uses a
 * small library-owned scratch per device: concurrent calls on one device
 * must be serialised (the reference's module-global scratch, likewise).  */
int hl_gpu_argmax(const float* logits, int n_vocab, int32_t* result,
                  void* stream);

/* As hl_gpu_argmax, but the index goes to result_dev (device memory) and
 * nothing waits for the stream (for graph capture and pipelined decode).
 * Extends the reference.                                                  */
int hl_argmax_async(const float* logits, int n_vocab, int32_t* result_dev,
                    void* stream);

/* gpuEmbedding (naive.nim:2975-3001): dst[e*nTokens + t] =
 * weight[tokenIds[t]*nEmb + e] for e < nEmb, t < nTokens (fp32; token ids
 * in device memory).  A token id outside [0, nVocab) gives a NaN column
 * (the reference reads out of bounds).                                    */
int hl_gpu_embedding(float* dst, const float* weight, const int32_t* token_ids,
                     int n_emb, int n_tokens, int n_vocab, void* stream);

/* ------------------------------------------------------------------------ */
/* Batched / typed API (extends the reference: B sequences, fp16/bf16 KV)   */
/* ------------------------------------------------------------------------ */

/* KV-cache layouts (the kv_layout fields below; 0 when a caller leaves the
 * field zero).  HL_KV_COLMAJOR is the reference's cache: per sequence,
 * [Hkv*D, max_len] column-major, element (row h*D + d, column t) at
 * (h*D + d)*max_len + t (naive.nim:3565-3567, 3239).  HL_KV_TILED32 keeps
 * each kv head's block the same size and at the same place, h*D*max_len,
 * but stores it as max_len/32 tiles of [D][32]: element (d, t) of head h at
 * h*D*max_len + ((t/32)*D + d)*32 + t%32, so 32 columns of a head are one
 * contiguous run (8 KB at D = 128 in fp16/bf16) instead of D runs of 64
 * bytes max_len apart.  Tiled caches: fp16/bf16 only, max_len % 32 == 0,
 * 16-byte aligned, batch stride a multiple of 8 elements.  No counterpart
 * in the reference (docs/future.md:38-43 lists cache layouts as future
 * work); a layout for callers that own their cache format.                */
#define HL_KV_COLMAJOR 0
#define HL_KV_TILED32 1
/* HL_KV_PAGED32: the caches are pools of 32-position pages.  Page p holds
 * positions 32j .. 32j+31 of one sequence for every kv head, as [Hkv][D][32]:
 * element (d, t) of head h of sequence b is at
 *   block_table[b * blocks_per_seq + t/32] * (Hkv*D*32) + (h*D + d)*32 + t%32
 * (block_table: device int32).  Each head's 32 columns are the same [D][32]
 * tile as in HL_KV_TILED32.  Same requirements as the tiled layout
 * (fp16/bf16/fp8, max_len % 32 == 0 with max_len/32 <= blocks_per_seq,
 * 16-byte aligned pools); cache_batch_stride is ignored.  A page is written
 * by the steps and prefills of its sequence only; pages of positions at or
 * past a sequence's length are never read.                                 */
#define HL_KV_PAGED32 2

typedef struct hl_decode_args {
  int batch;                    /* B >= 1                                        */
  int n_head;                   /* Hq                                            */
  int n_head_kv;                /* Hkv, Hq % Hkv == 0                             */
  int head_dim;                 /* D                                             */
  int kv_dtype;                 /* HL_F32 | HL_F16 | HL_BF16                      */
  int max_len;                  /* cache columns (cacheCols)                     */
  int seq_len;                  /* attention length L = pos+1 (max over B when
                                   seq_lens is given)                           */
  const int* seq_lens;          /* optional device int[B] of per-sequence L       */
  long long cache_batch_stride; /* elements between sequences (0 = dense)        */
  const float* q;               /* device [B][Hq*D] fp32                         */
  const void* k_cache;          /* device [B][Hkv*D, max_len] kv_dtype           */
  const void* v_cache;
  float* out;                   /* device [B][Hq*D] fp32                         */
  float scale;                  /* 0 -> 1/sqrtf(D) (naive.nim:3374)              */
  int num_splits;               /* 0 -> chosen to fill the GPU                   */
  int kv_layout;                /* HL_KV_COLMAJOR (0) | HL_KV_TILED32 | PAGED32  */
  const int* block_table;       /* HL_KV_PAGED32: device int[B][blocks_per_seq]  */
  int blocks_per_seq;
} hl_decode_args;

/* Workspace bytes hl_attn_decode needs for these args: 4-byte arrival
 * counters, one per (sequence, kv head, pair of query heads of its group),
 * rounded up to 256 bytes,
 * then the split-K partials (running max, sum and D accumulators per split
 * per query head).  The counters must be zero before the first call
 * (hl_attn_decode_workspace_init on the freshly allocated workspace); every
 * call leaves its counters zero again, so the workspace may be reused by
 * calls with any split count as long as it holds no other data in between.
 * A call whose counter region (batch x kv heads x head chunks) is larger than
 * the previous call's on the same workspace needs another init first.
 * Calls that overlap in time (e.g. on two streams) must not share a
 * workspace.  Returns 0 when the plan needs no workspace (a single split). */
size_t hl_attn_decode_workspace_bytes(const hl_decode_args* a);

/* Zero-fills `bytes` of workspace on `stream` (a kernel, not a memset, so it
 * may be captured in a HIP graph).  Call once after allocating a decode
 * workspace.  No counterpart in the reference (its decode has no split-K
 * workspace).                                                             */
int hl_attn_decode_workspace_init(void* workspace, size_t bytes, void* stream);

/* Decode attention for B sequences (the batched form of
 * gpuAttentionDecode, naive.nim:3369-3383).  `workspace` is device memory
 * of at least hl_attn_decode_workspace_bytes(a) bytes (in HippoLeap:
 * GpuContext.attnScratch, backend_types.nim:125-126).                    */
int hl_attn_decode(const hl_decode_args* a, void* workspace, size_t ws_bytes,
                   void* stream);

typedef struct hl_rope_store_args {
  int batch, n_head_q, n_head_kv, head_dim;
  int rope_dim;                 /* 0 -> head_dim; dims >= rope_dim pass through */
  int rope_style;               /* HL_ROPE_HALF_SPLIT | HL_ROPE_INTERLEAVED      */
  float rope_base;              /* theta base, used when use_installed_theta==0  */
  int use_installed_theta;      /* 1 -> table from hl_set_rope_theta            */
  int kv_dtype, max_len;
  long long cache_batch_stride; /* 0 = dense                                     */
  float* q;                     /* device [B][Hq*D] fp32, rotated in place       */
  float* k;                     /* device [B][Hkv*D] fp32, normed+rotated in place*/
  const float* v;               /* device [B][Hkv*D] fp32                        */
  void* k_cache;                /* device [B][Hkv*D, max_len]                   */
  void* v_cache;
  const int* positions;         /* optional device int[B]; else `pos` for all   */
  int pos;
  const float* q_norm_w;        /* optional device [D]: qkNorm before RoPE       */
  const float* k_norm_w;        /* optional device [D]                           */
  float eps;
  int kv_layout;                /* HL_KV_COLMAJOR (0) | HL_KV_TILED32 | PAGED32  */
  const int* block_table;       /* HL_KV_PAGED32: device int[B][blocks_per_seq]  */
  int blocks_per_seq;
} hl_rope_store_args;

/* One launch for the new token of B sequences: optional qkNorm of q and k
 * (naive.nim:4697-4700), RoPE at the position (naive.nim:3046-3073), and
 * the write of k and v into cache column `pos` in kv_dtype with
 * round-to-nearest-even (the drop-in for gpuQkNorm + gpuFusedRopeStoreKV,
 * naive.nim:2918-2926, 3149-3223).  Fails with HL_ECAPACITY when a
 * position is >= max_len (the "KV cache full" check, naive.nim:4598-4599,
 * for the host `pos`; device positions are not inspected).               */
int hl_rope_store_decode(const hl_rope_store_args* a, void* stream);

/* One decode step for the new token of B sequences: the result of
 * hl_rope_store_decode(rs) followed by hl_attn_decode(at) on the same
 * stream (identical cache contents and output), in one launch for fp16/bf16
 * KV (two for fp32).  It replaces the reference's per-layer sequence
 * gpuQkNorm + gpuFusedRopeStoreKV + gpuAttentionDecode (naive.nim:4697-4700,
 * 3149-3223, 3369-3383).  rs and at must describe the same tensors
 * (at->q == rs->q, same caches, shapes, dtype and stride); at->seq_lens must
 * be null: sequence b attends over positions[b] + 1 columns (rs->pos + 1
 * when rs->positions is null, and then at->seq_len must equal rs->pos + 1;
 * with positions, at->seq_len is the longest such length, used only to plan
 * the splits).  Unlike hl_rope_store_decode, q and k are read only when the
 * step runs as one launch; with fp32 KV they are rotated in place, so treat
 * their contents as unspecified afterwards.  The workspace follows the rules
 * of hl_attn_decode's, sized by hl_decode_step_workspace_bytes.          */
size_t hl_decode_step_workspace_bytes(const hl_rope_store_args* rs, const hl_decode_args* at);
int hl_decode_step(const hl_rope_store_args* rs, const hl_decode_args* at, void* workspace,
                   size_t ws_bytes, void* stream);

typedef struct hl_prefill_args {
  int n_head, n_head_kv, head_dim, seq_len;
  int io_dtype;                 /* dtype of q/k/v/out: HL_F32|HL_F16|HL_BF16     */
  const void* q;                /* device col-major [Hq*D, T]                    */
  const void* k;                /* device col-major [Hkv*D, T]                   */
  const void* v;
  void* out;                    /* device col-major [Hq*D, T] out_dtype          */
  /* fused before attention (naive.nim:4067-4076)                              */
  const float* q_norm_w;        /* optional [D] (qkNorm, Qwen3)                  */
  const float* k_norm_w;
  float eps;
  int apply_rope;               /* 1 -> RoPE of q and k at positions start_pos+p */
  int rope_dim;                 /* 0 -> head_dim                                 */
  int rope_style;
  float rope_base;
  int use_installed_theta;
  /* fused KV-cache write (naive.nim:4075-4076); k_cache == NULL skips it      */
  void* k_cache;
  void* v_cache;
  int kv_dtype;
  int max_len;
  int start_pos;
  float scale;                  /* 0 -> 1/sqrtf(D)                               */
  int write_back_qk;            /* 1 (fp32 only): leave normed+roped q,k in the
                                   q/k buffers, as the reference's in-place ops do*/
  int out_dtype;                /* dtype of `out`: HL_F32 (default, the
                                   reference's fp32 act1) or, for fp16/bf16
                                   io, HL_F16 / HL_BF16 (RNE of the fp32 value) */
  int kv_layout;                /* of k_cache/v_cache: HL_KV_COLMAJOR (0) |
                                   HL_KV_TILED32 | HL_KV_PAGED32                */
  const int* block_table;       /* HL_KV_PAGED32: device int[max_len/32], this
                                   sequence's pages                             */
} hl_prefill_args;

/* Workspace hl_attn_prefill needs for these args (0: none).  It holds the
 * MFMA path's fp16 operands and fallback buffers, or, for fp32 activations,
 * the roped Q and K when RoPE / qkNorm run, and the K/V
 * split images (8 bytes per K and V element, padded to 64-token tiles).   */
size_t hl_attn_prefill_workspace_bytes(const hl_prefill_args* a);

/* Causal prefill with the pre-attention ops fused: qkNorm -> RoPE -> KV
 * cache write -> flash attention (bf16/fp16: MFMA; fp32: vector ALU).
 * Replaces naive.nim:4067-4078 for one attention layer.  Errors:
 * HL_EINVAL for shapes / GQA, HL_ECAPACITY for start_pos+T > max_len
 * (naive.nim:3975-3976).                                                  */
int hl_attn_prefill(const hl_prefill_args* a, void* workspace, size_t ws_bytes,
                    void* stream);

/* The MFMA prefill (bf16/fp16 activations) rounds Q * scale, K and V, after
 * qkNorm and RoPE, to fp16 operands.  A value of magnitude >= 65520 has no
 * fp16 form; the kernels record such a value in the call's workspace, and
 * two gated kernels that every MFMA prefill launches after its flash kernel
 * then recompute the whole output from the original activations in fp32
 * (fp32 operands and accumulation, as the reference's fp32 prefill,
 * naive.nim:3385-3464).  While nothing overflows they return at once.  So
 * hl_attn_prefill's output is valid over the whole range of its inputs with
 * no call to this function, also under stream capture.  This function only
 * reports, for tests and diagnostics, whether the last hl_attn_prefill on
 * `workspace` with these args took that fallback: it waits for `stream`
 * and sets *ran to 1 or 0 (always 0 for fp32 activations).  Under stream
 * capture it returns HL_ECAPTURE.  No counterpart in the reference.
 * The record is 16 bytes at the end of the workspace; each call retires its
 * own mark, so it needs no initialisation (zero-filled, or left by an
 * earlier prefill; arbitrary bytes can at worst send one call through the
 * fallback, with the same result).  Calls that share a workspace must not
 * overlap (one stream, as everywhere in this library).                   */
int hl_attn_prefill_fallback_ran(const hl_prefill_args* a, const void* workspace, int* ran,
                                 void* stream);

/* Reads cache columns [col0, col0+ncols) of a [rows, max_len] cache of
 * kv_dtype into fp32 dst[rows, ncols] (exact upcast; halfToFloat semantics,
 * quant.nim:78-96).  Debug / host-mirror helper (KvCache.k, types:41-49). */
int hl_kv_cache_to_f32(float* dst, const void* cache, int kv_dtype, int rows,
                       int max_len, int col0, int ncols, void* stream);

/* ------------------------------------------------------------------------ */
/* Elementwise drop-ins of the decode step (fp32).                           */
/* ------------------------------------------------------------------------ */

/* gpuSiluMul (naive.nim:2179-2193): dst[i] = gate[i] * (1/(1 + expf(-gate[i])))
 * * up[i] for i < n.  dst may alias gate or up.                           */
int hl_gpu_silu_mul(float* dst, const float* gate, const float* up, int n,
                    void* stream);

/* gpuAdd (naive.nim:2132-2145): dst[i] = a[i] + b[i].  dst may alias a or b. */
int hl_gpu_add(float* dst, const float* a, const float* b, int n, void* stream);

/* gpuFusedGateUpSiluQ4K / gpuFusedGateUpSiluQ3K (naive.nim:1905-1920,
 * 1693-1708) for any GGUF type of hl_gpu_linear_col_quant: dst[wRows] =
 * silu(gate . x) * (up . x), both matrices [wRows, wCols] of quant_type, in
 * one launch (silu as gpuSiluMul).  x must be 16-byte aligned and the
 * weights aligned to their blocks (16 bytes for F16, Q4_K, Q5_K; 4 for
 * Q2_K; 2 otherwise): HL_EINVAL if not.                                    */
int hl_gpu_fused_gate_up_silu_quant(float* dst, const float* x, const void* gate_q,
                                    const void* up_q, int w_cols, int w_rows,
                                    int quant_type, void* stream);
int hl_gpu_fused_gate_up_silu_q4k(float* dst, const float* x, const void* gate_q,
                                  const void* up_q, int w_cols, int w_rows, void* stream);
int hl_gpu_fused_gate_up_silu_q3k(float* dst, const float* x, const void* gate_q,
                                  const void* up_q, int w_cols, int w_rows, void* stream);

/* gpuFusedKVLinearQ4K / gpuFusedKVLinearQ2KQ3K (naive.nim:1799-1814,
 * 853-868) for any GGUF types: k_dst = k_q . x, v_dst = v_q . x (both
 * [wRows, wCols]); one launch when the types match and the pointers allow
 * it, two otherwise.                                                      */
int hl_gpu_fused_kv_linear_quant(float* k_dst, float* v_dst, const float* x, const void* k_q,
                                 const void* v_q, int w_cols, int w_rows, int k_type,
                                 int v_type, void* stream);
int hl_gpu_fused_kv_linear_q4k(float* k_dst, float* v_dst, const float* x, const void* k_q,
                               const void* v_q, int w_cols, int w_rows, void* stream);
int hl_gpu_fused_kv_linear_q2k_q3k(float* k_dst, float* v_dst, const float* x,
                                   const void* k_q, const void* v_q, int w_cols,
                                   int w_rows, void* stream);

/* ------------------------------------------------------------------------ */
/* One greedy decode step of a dense decoder (forwardDecodeToken for layers   */
/* of kind lkAttentionFfn, naive.nim:4592-4760, 5520-5545).                  */
/* ------------------------------------------------------------------------ */

/* A weight matrix: w_type 0 = fp32 row-major [rows, cols] (gpuLinearCol),
 * otherwise a GGUF type of hl_gpu_linear_col_quant.                        */
typedef struct {
  const float* attn_norm;   /* [n_emb]                                       */
  const float* q_norm;      /* [head_dim] or NULL (no qk-norm)               */
  const float* k_norm;      /* [head_dim] or NULL                            */
  const float* ffn_norm;    /* [n_emb]                                       */
  const void* wq;           /* [n_head*head_dim, n_emb]                      */
  const void* wk;           /* [n_head_kv*head_dim, n_emb]                   */
  const void* wv;           /* [n_head_kv*head_dim, n_emb]                   */
  const void* wo;           /* [n_emb, n_head*head_dim]                      */
  const void* w_gate;       /* [n_ff, n_emb]                                 */
  const void* w_up;         /* [n_ff, n_emb]                                 */
  const void* w_down;       /* [n_emb, n_ff]                                 */
  int wq_type, wk_type, wv_type, wo_type, w_gate_type, w_up_type, w_down_type;
  float* k_cache;           /* [n_head_kv*head_dim, max_len] fp32 (as a1)    */
  float* v_cache;
} hl_layer_desc;

typedef struct {
  int n_layer, n_emb, n_head, n_head_kv, head_dim;
  int rope_dim;                /* <= 0 -> head_dim (the reference's ropeDim)  */
  int n_ff, n_vocab, max_len;
  float rms_eps, rope_base;
  const float* tok_emb;        /* [n_vocab, n_emb] fp32                      */
  const float* output_norm;    /* [n_emb]                                    */
  const void* output;          /* [n_vocab, n_emb]                           */
  int output_type;
  const hl_layer_desc* layers; /* host array of n_layer                      */
} hl_model_desc;

/* Caller-owned device scratch (the reference's x, xNorm and tmp buffers):
 * x [n_emb]; x_norm [max(n_emb, n_head*head_dim)]; tmp0 [max(n_emb,
 * n_head*head_dim, n_ff)]; tmp1, tmp2 [max(n_head_kv*head_dim, n_ff)].    */
typedef struct {
  float* x;
  float* x_norm;
  float* tmp0;
  float* tmp1;
  float* tmp2;
} hl_decode_scratch;

/* Runs the token at *token_dev (device int32) through every layer at
 * position pos, writing the K/V column pos of each layer's cache, the
 * logits [n_vocab] and the greedy next token to *next_token_dev (device;
 * nothing waits for the stream, so next_token_dev can be the next call's
 * token_dev).  The reference's step, in its order: embedding; rmsnorm;
 * per layer Q/K/V projections (one launch when the three weights share a
 * quantized type, as K/V pairs and gate/up pairs are), qk-norm, RoPE,
 * K/V store, attention, O projection, residual + ffn norm, gate/up,
 * SiLU * up (the residual and norm inside the gate/up launch when that runs
 * Q4_K on the matrix cores), down, residual + next layer's norm; final norm, output
 * projection, argmax.  Sets the process-wide RoPE table
 * (hl_set_rope_theta) on every call: steps of models with different RoPE
 * parameters must not run concurrently (the reference's theta table is
 * module-global too).                                                     */
int hl_forward_decode_token(const hl_model_desc* model, const hl_decode_scratch* scratch,
                            const int32_t* token_dev, int pos, float* logits,
                            int32_t* next_token_dev, void* stream);

/* ------------------------------------------------------------------------ */
/* The backend contract over a KV-cache descriptor: initKvCache,             */
/* forwardPrefill and forwardDecodeToken (naive.nim:3912-3931, 3967-4590,    */
/* 4592-4760) for models whose layers are all of kind lkAttentionFfn.        */
/* ------------------------------------------------------------------------ */

/* A model's KV cache (KvCache / GpuKvCache, backend_types.nim:28-49) with a
 * storage dtype and layout, which the reference's cache lacks (its caches
 * are fp32 [kvDim, maxLen]).  The caller owns the buffers: per layer one K
 * and one V cache of hl_kv_cache_bytes() bytes each, in device memory.     */
typedef struct hl_kv_cache_desc {
  int n_layer, n_head_kv, head_dim, max_len;
  int kv_dtype;                 /* HL_F32 (the reference's) | HL_F16 | HL_BF16 |
                                   HL_FP8 (tiled or paged layouts only)         */
  int kv_layout;                /* HL_KV_COLMAJOR | HL_KV_TILED32 | PAGED32      */
  void* const* k;               /* host array [n_layer] of device caches        */
  void* const* v;
  const int* block_table;       /* HL_KV_PAGED32: device int[blocks_per_seq]    */
  int blocks_per_seq;
  int cur_len;                  /* positions written (curLen): prefill sets it,
                                   each decode step advances it by one          */
} hl_kv_cache_desc;

/* Bytes of one layer's K (or V) cache in this dtype and layout: the
 * reference's newTensor(@[kvDim, maxLen]) of initKvCache (naive.nim:
 * 3926-3927), which is n_head_kv * head_dim * max_len fp32 values.  0 for
 * a combination the library does not build.                               */
size_t hl_kv_cache_bytes(int n_head_kv, int head_dim, int max_len, int kv_dtype, int kv_layout);

/* The layout initKvCache should allocate for this dtype: HL_KV_TILED32
 * for fp16/bf16/fp8 caches whose max_len is a multiple of 32 (decode
 * streams each 32-column tile as one contiguous run: the c5 step at 67-70%
 * of HBM against 63% column-major), HL_KV_COLMAJOR otherwise (fp32, the
 * reference's own cache, or an odd max_len).                              */
int hl_kv_cache_preferred_layout(int kv_dtype, int max_len);

/* initKvCache (naive.nim:3912-3931) for a cache descriptor the caller has
 * filled: checks it against the model (layer count, kv heads, head dim,
 * dtype/layout/alignment rules of the decode and prefill entry points, a
 * cache pointer per layer) and sets cur_len = 0.                           */
int hl_kv_cache_init(hl_kv_cache_desc* cache, const hl_model_desc* model);

/* Activation scratch of the forward entry points (the reference's act0/1
 * and scratch0..2, sized for max_tokens columns) plus the attention
 * workspace, all caller-owned device memory.  Nothing below allocates.     */
typedef struct {
  int max_tokens;               /* columns the activation buffers hold (>= 1) */
  float* x;                     /* [n_emb * max_tokens]                         */
  float* x_norm;                /* [max(n_emb, n_head*head_dim) * max_tokens]  */
  float* tmp0;                  /* [max(n_emb, n_head*head_dim, n_ff) * max_tokens] */
  float* tmp1;                  /* [max(n_head_kv*head_dim, n_ff) * max_tokens] */
  float* tmp2;                  /* [max(n_head_kv*head_dim, n_ff) * max_tokens] */
  void* workspace;              /* hl_forward_workspace_bytes() bytes, 16-byte
                                   aligned, zero-filled once with
                                   hl_attn_decode_workspace_init                */
  size_t workspace_bytes;
} hl_forward_scratch;

/* Attention workspace bytes that prefills of up to max_tokens tokens and
 * decode steps at every position < max_len need with this cache.          */
size_t hl_forward_workspace_bytes(const hl_model_desc* model, const hl_kv_cache_desc* cache,
                                  int max_tokens);

/* forwardPrefill (naive.nim:3967-4590), lkAttentionFfn layers: the
 * n_tokens device int32 tokens at positions 0 .. n_tokens-1 through every
 * layer (rmsnorm, Q/K/V projections, qk-norm, RoPE, K/V into the cache,
 * causal attention, O projection, residual, rmsnorm, gate/up, SiLU * up,
 * down, residual), then the final norm and the output projection into
 * logits [n_vocab, n_tokens] (device, col-major, the reference's result
 * tensor).  Sets cache->cur_len = n_tokens.  Weights are fp32 (type 0), as
 * the reference's prefill takes them (it uploads fp32 copies); a quantized
 * weight returns HL_EUNSUPPORTED.  Errors: the reference's ValueErrors
 * (GQA, empty prompt, "prefill exceeds KV cache capacity"), checked with
 * every pointer and shape before the first launch.                        */
int hl_forward_prefill(const hl_model_desc* model, hl_kv_cache_desc* cache,
                       const hl_forward_scratch* scratch, const int32_t* tokens_dev,
                       int n_tokens, float* logits, void* stream);

/* forwardDecodeToken (naive.nim:4592-4760, 5520-5545): the token at
 * *token_dev at position cache->cur_len (the K/V column written), logits
 * [n_vocab] and the greedy next token into *next_token_dev, then
 * cache->cur_len += 1.  fp16/bf16/fp8 caches run each layer's qk-norm,
 * RoPE, cache write and attention as one launch (hl_decode_step); fp32
 * caches run the reference's sequence.  Weights fp32 or any GGUF type of
 * hl_gpu_linear_col_quant.  "KV cache full" (HL_ECAPACITY) when cur_len ==
 * max_len.  Nothing allocates or waits for the stream.                    */
int hl_forward_decode(const hl_model_desc* model, hl_kv_cache_desc* cache,
                      const hl_forward_scratch* scratch, const int32_t* token_dev,
                      float* logits, int32_t* next_token_dev, void* stream);

/* forwardDecodeTokenTimed (megakernel.nim:2514-2529, called by
 * inference.nim:80-84): hl_forward_decode bracketed by two hipEvents on
 * `stream` (created once per device and kept), then waits for the stream
 * and returns the greedy next token in host *next_token (also left in
 * *next_token_dev) and the GPU time between the events, in ms, in *gpu_ms.
 * The events bracket the embedding through the argmax, as the reference's
 * bracket forwardDecodeGpu + gpuArgmax.  It waits, so under stream capture
 * it returns HL_ECAPTURE (capture hl_forward_decode itself and time the
 * graph).  cache->cur_len advances as in hl_forward_decode.              */
int hl_forward_decode_timed(const hl_model_desc* model, hl_kv_cache_desc* cache,
                            const hl_forward_scratch* scratch, const int32_t* token_dev,
                            float* logits, int32_t* next_token_dev, int32_t* next_token,
                            float* gpu_ms, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HL_ATTN_H */
