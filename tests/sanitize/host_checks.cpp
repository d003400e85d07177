// Host-side validation and planning of libhl_attn under AddressSanitizer and
// UndefinedBehaviorSanitizer (no GPU; built by tests/test_host_sanitize.py
// with the device passes left out).  Every call below returns before any
// HIP launch: argument checks, workspace-size planning over a sweep of
// shapes, and the "workspace too small by one byte" refusal that every
// entry point applies after planning, which exercises the same offset
// arithmetic the kernels trust.  Exit status 0 and no sanitizer report is
// the pass condition.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "hl_attn.h"

static int g_fail = 0;
static void* const FAKE = (void*)(uintptr_t)(1 << 20);  // aligned, never dereferenced

#define EXPECT(cond, ...)                          \
  do {                                             \
    if (!(cond)) {                                 \
      std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      std::fprintf(stderr, __VA_ARGS__);           \
      std::fprintf(stderr, " [%s]\n", hl_last_error()); \
      ++g_fail;                                    \
    }                                              \
  } while (0)

static hl_decode_args decode_args(int B, int hq, int hkv, int d, int dt, int M, int L, int layout, int splits) {
  hl_decode_args a;
  std::memset(&a, 0, sizeof(a));
  a.batch = B;
  a.n_head = hq;
  a.n_head_kv = hkv;
  a.head_dim = d;
  a.kv_dtype = dt;
  a.max_len = M;
  a.seq_len = L;
  a.q = (const float*)FAKE;
  a.k_cache = a.v_cache = FAKE;
  a.out = (float*)FAKE;
  a.num_splits = splits;
  a.kv_layout = layout;
  if (layout == HL_KV_PAGED32) {
    a.block_table = (const int*)FAKE;
    a.blocks_per_seq = M / 32;
  }
  return a;
}

static hl_rope_store_args rope_args(const hl_decode_args& at, int rope_dim, int style, bool norm) {
  hl_rope_store_args r;
  std::memset(&r, 0, sizeof(r));
  r.batch = at.batch;
  r.n_head_q = at.n_head;
  r.n_head_kv = at.n_head_kv;
  r.head_dim = at.head_dim;
  r.rope_dim = rope_dim;
  r.rope_style = style;
  r.rope_base = 5e5f;
  r.kv_dtype = at.kv_dtype;
  r.max_len = at.max_len;
  r.q = (float*)at.q;
  r.k = r.q + 4096;
  r.v = r.q + 8192;
  r.k_cache = (void*)at.k_cache;
  r.v_cache = (void*)at.v_cache;
  r.pos = at.seq_len - 1;
  r.q_norm_w = norm ? (const float*)FAKE : nullptr;
  r.k_norm_w = norm ? (const float*)FAKE : nullptr;
  r.eps = 1e-6f;
  r.kv_layout = at.kv_layout;
  r.block_table = at.block_table;
  r.blocks_per_seq = at.blocks_per_seq;
  return r;
}

static void decode_sweep() {
  const int Bs[] = {1, 3, 8, 16};
  const int heads[][2] = {{32, 4}, {32, 8}, {40, 2}, {16, 16}, {8, 1}, {64, 8}};
  const int Ds[] = {64, 128};
  const int Ls[] = {1, 17, 512, 2049, 32769, 131072};
  const int dts[] = {HL_F32, HL_F16, HL_BF16, HL_FP8};
  const int splits[] = {0, 1, 3, 64};
  int planned = 0;
  for (int B : Bs)
    for (auto& h : heads)
      for (int d : Ds)
        for (int L : Ls)
          for (int dt : dts)
            for (int layout = 0; layout < 3; ++layout)
              for (int sp : splits) {
                if (dt == HL_F32 && layout != HL_KV_COLMAJOR) continue;
                if (dt == HL_FP8 && layout == HL_KV_COLMAJOR) continue;
                const int M = layout == HL_KV_COLMAJOR ? L : (L + 31) / 32 * 32;
                hl_decode_args a = decode_args(B, h[0], h[1], d, dt, M, L, layout, sp);
                const size_t need = hl_attn_decode_workspace_bytes(&a);
                if (need > 0) {
                  EXPECT(hl_attn_decode(&a, FAKE, need - 1, nullptr) == HL_EINVAL,
                         "decode B%d H%d/%d D%d L%d dt%d lay%d sp%d: short workspace accepted", B, h[0], h[1], d, L,
                         dt, layout, sp);
                  ++planned;
                }
                if (dt == HL_F32 || sp != 0) continue;
                for (int norm = 0; norm < 2; ++norm) {
                  hl_rope_store_args r = rope_args(a, norm ? 0 : d / 2, norm, norm);
                  const size_t sneed = hl_decode_step_workspace_bytes(&r, &a);
                  if (sneed > 0)
                    EXPECT(hl_decode_step(&r, &a, FAKE, sneed - 1, nullptr) == HL_EINVAL,
                           "step B%d L%d: short workspace accepted", B, L);
                }
              }
  EXPECT(planned > 1000, "decode sweep planned only %d cases", planned);
}

static hl_prefill_args prefill_args(int hq, int hkv, int d, int T, int io, int rope, int rd, int style, bool norm,
                                    bool cache, int layout) {
  hl_prefill_args a;
  std::memset(&a, 0, sizeof(a));
  a.n_head = hq;
  a.n_head_kv = hkv;
  a.head_dim = d;
  a.seq_len = T;
  a.io_dtype = io;
  a.q = a.k = a.v = FAKE;
  a.out = FAKE;
  a.apply_rope = rope;
  a.rope_dim = rd;
  a.rope_style = style;
  a.rope_base = 5e5f;
  a.q_norm_w = norm ? (const float*)FAKE : nullptr;
  a.k_norm_w = norm ? (const float*)FAKE : nullptr;
  a.eps = 1e-6f;
  if (cache) {
    a.k_cache = a.v_cache = FAKE;
    a.kv_dtype = io == HL_F32 ? HL_F32 : HL_BF16;
    a.kv_layout = io == HL_F32 ? HL_KV_COLMAJOR : layout;
    a.max_len = (T + 31) / 32 * 32 + 64;
    if (a.kv_layout == HL_KV_PAGED32) a.block_table = (const int*)FAKE;
  }
  a.out_dtype = HL_F32;
  return a;
}

static void prefill_sweep() {
  const int heads[][2] = {{32, 4}, {32, 8}, {8, 2}, {40, 2}, {4, 4}};
  const int Ds[] = {64, 128};
  const int Ts[] = {1, 31, 64, 65, 512, 4096, 8191};
  const int ios[] = {HL_F32, HL_F16, HL_BF16};
  int planned = 0;
  for (auto& h : heads)
    for (int d : Ds)
      for (int T : Ts)
        for (int io : ios)
          for (int variant = 0; variant < 6; ++variant) {
            const int rope = variant != 0, rd = variant == 2 ? d / 2 : 0, style = variant == 3;
            const bool norm = variant >= 4, cache = variant != 1;
            const int layout = variant == 5 ? HL_KV_PAGED32 : (variant == 4 ? HL_KV_TILED32 : HL_KV_COLMAJOR);
            hl_prefill_args a = prefill_args(h[0], h[1], d, T, io, rope, rd, style, norm, cache, layout);
            const size_t need = hl_attn_prefill_workspace_bytes(&a);
            if (need > 0) {
              EXPECT(hl_attn_prefill(&a, FAKE, need - 1, nullptr) == HL_EINVAL,
                     "prefill H%d/%d D%d T%d io%d v%d: short workspace accepted", h[0], h[1], d, T, io, variant);
              ++planned;
            }
          }
  EXPECT(planned > 300, "prefill sweep planned only %d cases", planned);
}

static void reference_prechecks() {
  hl_decode_args a = decode_args(1, 6, 4, 64, HL_F16, 2049, 2049, 0, 0);
  EXPECT(hl_attn_decode(&a, nullptr, 0, nullptr) == HL_EINVAL, "GQA");
  EXPECT(std::strcmp(hl_last_error(), "GQA requires head_count divisible by head_count_kv") == 0, "GQA text");
  a = decode_args(1, 32, 8, 64, HL_F16, 2049, 2050, 0, 0);
  EXPECT(hl_attn_decode(&a, nullptr, 0, nullptr) == HL_ECAPACITY, "cache full");
  EXPECT(std::strcmp(hl_last_error(), "KV cache full") == 0, "cache full text");
  a = decode_args(1, 32, 8, 96, HL_F16, 2049, 2049, 0, 0);
  EXPECT(hl_attn_decode(&a, nullptr, 0, nullptr) == HL_EUNSUPPORTED, "head dim");
  a = decode_args(1, 32, 8, 64, HL_F16, 2049, 2049, 0, 0);
  a.q = nullptr;
  EXPECT(hl_attn_decode(&a, nullptr, 0, nullptr) == HL_EINVAL, "null q");
  EXPECT(hl_gpu_attention_decode((float*)FAKE, (const float*)FAKE, (const float*)FAKE, (const float*)FAKE, 32, 4,
                                 64, 513, 512, nullptr) == HL_ECAPACITY,
         "drop-in cache full");
  hl_prefill_args p = prefill_args(32, 8, 128, 0, HL_BF16, 0, 0, 0, false, false, 0);
  EXPECT(hl_attn_prefill(&p, nullptr, 0, nullptr) == HL_EINVAL, "empty prefill");
  EXPECT(std::strcmp(hl_last_error(), "prefill requires at least one token") == 0, "empty text");
  p = prefill_args(32, 8, 128, 4096, HL_BF16, 0, 0, 0, false, true, 0);
  p.max_len = 4095;
  EXPECT(hl_attn_prefill(&p, nullptr, 0, nullptr) == HL_ECAPACITY, "prefill capacity");
  EXPECT(std::strcmp(hl_last_error(), "prefill exceeds KV cache capacity") == 0, "capacity text");
  // a tiled cache needs max_len % 32 == 0
  a = decode_args(2, 32, 4, 128, HL_BF16, 1000, 900, HL_KV_TILED32, 0);
  EXPECT(hl_attn_decode(&a, nullptr, 0, nullptr) == HL_EINVAL, "tiled max_len");
  // theta tables: every supported rope_dim, and refusals
  std::vector<float> th(256);
  for (int rd = 2; rd <= 256; rd += 2) EXPECT(hl_rope_theta_table(th.data(), rd, 1e4f) == HL_OK, "theta %d", rd);
  EXPECT(hl_rope_theta_table(th.data(), 3, 1e4f) != HL_OK, "odd rope dim");
  EXPECT(hl_rope_theta_table(th.data(), 1024, 1e4f) != HL_OK, "rope dim too large");
}

static void forward_checks() {
  const int n_layer = 3;
  std::vector<hl_layer_desc> layers(n_layer);
  std::memset(layers.data(), 0, sizeof(hl_layer_desc) * n_layer);
  for (auto& L : layers) {
    L.attn_norm = L.ffn_norm = (const float*)FAKE;
    L.wq = L.wk = L.wv = L.wo = L.w_gate = L.w_up = L.w_down = FAKE;
  }
  hl_model_desc m;
  std::memset(&m, 0, sizeof(m));
  m.n_layer = n_layer;
  m.n_emb = 256;
  m.n_head = 8;
  m.n_head_kv = 2;
  m.head_dim = 64;
  m.n_ff = 512;
  m.n_vocab = 1000;
  m.max_len = 96;
  m.rms_eps = 1e-5f;
  m.rope_base = 1e4f;
  m.tok_emb = m.output_norm = (const float*)FAKE;
  m.output = FAKE;
  m.layers = layers.data();
  std::vector<void*> caches(n_layer, FAKE);
  const int dts[] = {HL_F32, HL_F16, HL_BF16, HL_FP8};
  for (int dt : dts)
    for (int layout = 0; layout < 3; ++layout) {
      if ((dt == HL_F32 && layout) || (dt == HL_FP8 && !layout)) continue;
      EXPECT(hl_kv_cache_bytes(2, 64, 96, dt, layout) > 0, "cache bytes dt%d lay%d", dt, layout);
      hl_kv_cache_desc c;
      std::memset(&c, 0, sizeof(c));
      c.n_layer = n_layer;
      c.n_head_kv = 2;
      c.head_dim = 64;
      c.max_len = 96;
      c.kv_dtype = dt;
      c.kv_layout = layout;
      c.k = c.v = caches.data();
      if (layout == HL_KV_PAGED32) {
        c.block_table = (const int*)FAKE;
        c.blocks_per_seq = 3;
      }
      EXPECT(hl_kv_cache_init(&c, &m) == HL_OK, "cache init dt%d lay%d", dt, layout);
      for (int T : {1, 7, 96}) {
        const size_t need = hl_forward_workspace_bytes(&m, &c, T);
        EXPECT(need > 0, "forward workspace dt%d T%d", dt, T);
        hl_forward_scratch s;
        std::memset(&s, 0, sizeof(s));
        s.max_tokens = T;
        s.x = s.x_norm = s.tmp0 = s.tmp1 = s.tmp2 = (float*)FAKE;
        s.workspace = FAKE;
        s.workspace_bytes = need - 1;
        int32_t tok = 0;
        float ms = 0.f;
        if (T == 1) {
          EXPECT(hl_forward_decode_timed(&m, &c, &s, (const int32_t*)FAKE, (float*)FAKE, (int32_t*)FAKE, nullptr,
                                         &ms, nullptr) == HL_EINVAL,
                 "timed decode null token");
          EXPECT(hl_forward_decode_timed(&m, &c, &s, (const int32_t*)FAKE, (float*)FAKE, (int32_t*)FAKE, &tok,
                                         nullptr, nullptr) == HL_EINVAL,
                 "timed decode null time");
        }
        if (dt == HL_F32 || layout != HL_KV_PAGED32) {
          c.cur_len = 0;
          EXPECT(hl_forward_prefill(&m, &c, &s, (const int32_t*)FAKE, T, (float*)FAKE, nullptr) == HL_EINVAL,
                 "forward prefill short workspace dt%d T%d", dt, T);
        }
      }
      c.cur_len = 96;
      hl_forward_scratch s;
      std::memset(&s, 0, sizeof(s));
      s.max_tokens = 1;
      s.x = s.x_norm = s.tmp0 = s.tmp1 = s.tmp2 = (float*)FAKE;
      s.workspace = FAKE;
      s.workspace_bytes = hl_forward_workspace_bytes(&m, &c, 1);
      EXPECT(hl_forward_decode(&m, &c, &s, (const int32_t*)FAKE, (float*)FAKE, (int32_t*)FAKE, nullptr) ==
                 HL_ECAPACITY,
             "forward decode on a full cache dt%d", dt);
    }
  m.n_head = 6;
  m.n_head_kv = 4;
  hl_kv_cache_desc c;
  std::memset(&c, 0, sizeof(c));
  c.n_layer = n_layer;
  c.n_head_kv = 4;
  c.head_dim = 64;
  c.max_len = 96;
  c.k = c.v = caches.data();
  EXPECT(hl_kv_cache_init(&c, &m) == HL_EINVAL, "GQA model refused");
}

int main() {
  reference_prechecks();
  decode_sweep();
  prefill_sweep();
  forward_checks();
  if (g_fail) {
    std::fprintf(stderr, "%d host checks failed\n", g_fail);
    return 1;
  }
  std::printf("host checks passed\n");
  return 0;
}
