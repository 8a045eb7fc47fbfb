// extern "C" entry points declared in include/es_decode.h.
#include "es_decode.h"

#include <hip/hip_runtime.h>

#include <cstring>
#include <string>

#include "es_checkpoint.hpp"
#include "es_engine.hpp"
#include "es_kernels.hpp"
#include "es_weights.hpp"

struct es_engine {
  es::Engine* impl;
};

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ES_OK;
  if (e == hipErrorInvalidValue) return fail(ES_ERR_INVALID, std::string(what) + ": invalid arguments or shapes");
  return fail(ES_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

bool to_q4(const es_q4* in, es::Q4* out) {
  if (!in) return false;
  *out = es::Q4{in->codes, in->scales, in->biases, in->n, in->k};
  return in->codes && in->scales && in->biases && in->n > 0 && in->k > 0;
}

hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

int engine_rc(int rc, const std::string& err) {
  if (rc == 0) return ES_OK;
  if (rc == 3) return fail(ES_ERR_CANCELLED, err);
  if (rc == 2) return fail(ES_ERR_DEVICE, err);
  return fail(ES_ERR_INVALID, err);
}

}  // namespace

extern "C" {

const char* es_last_error(void) { return g_error.c_str(); }

// ---- plumbing ----
int es_device_count(int* count) {
  if (!count) return fail(ES_ERR_INVALID, "null count");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) n = 0;
  *count = n;
  return ES_OK;
}
int es_device_name(int device, char* buf, int len) {
  if (!buf || len <= 0) return fail(ES_ERR_INVALID, "null buffer");
  hipDeviceProp_t p;
  if (int rc = hip_status(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties")) return rc;
  std::snprintf(buf, len, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
  return ES_OK;
}
int es_set_device(int device) { return hip_status(hipSetDevice(device), "hipSetDevice"); }
int es_malloc(void** ptr, size_t bytes) {
  if (!ptr) return fail(ES_ERR_INVALID, "null ptr");
  return hip_status(hipMalloc(ptr, bytes ? bytes : 1), "hipMalloc");
}
int es_free(void* ptr) { return hip_status(hipFree(ptr), "hipFree"); }
int es_memcpy_htod(void* dst, const void* src, size_t bytes) {
  return hip_status(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
}
int es_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
  return hip_status(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}
int es_memset(void* dst, int value, size_t bytes) {
  return hip_status(hipMemset(dst, value, bytes), "hipMemset");
}
int es_copy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes % 16 != 0) return fail(ES_ERR_INVALID, "es_copy_d2d: bytes must be a multiple of 16");
  return hip_status(es::launch_copy16(dst, src, bytes, S(stream)), "es_copy_d2d");
}
int es_time_read(const void* src, size_t bytes, void* out, size_t out_bytes, int reps, double* ms_avg) {
  if (!ms_avg || !src || !out || reps <= 0 || bytes == 0 || bytes % es::read_granule() != 0 ||
      out_bytes < es::read_out_bytes())
    return fail(ES_ERR_INVALID, "es_time_read: bad arguments");
  hipEvent_t e0, e1;
  if (int rc = hip_status(hipEventCreate(&e0), "hipEventCreate")) return rc;
  if (int rc = hip_status(hipEventCreate(&e1), "hipEventCreate")) return rc;
  int rc = hip_status(es::launch_read(src, bytes, out, nullptr), "read warmup");
  if (!rc) rc = hip_status(hipEventRecord(e0, nullptr), "hipEventRecord");
  for (int i = 0; i < reps && !rc; ++i) rc = hip_status(es::launch_read(src, bytes, out, nullptr), "read");
  if (!rc) rc = hip_status(hipEventRecord(e1, nullptr), "hipEventRecord");
  if (!rc) rc = hip_status(hipEventSynchronize(e1), "hipEventSynchronize");
  float ms = 0.0f;
  if (!rc) rc = hip_status(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (!rc) *ms_avg = ms / reps;
  return rc;
}
int es_time_copy_d2d(void* dst, const void* src, size_t bytes, int reps, double* ms_avg) {
  if (!ms_avg || reps <= 0 || bytes % 16 != 0) return fail(ES_ERR_INVALID, "es_time_copy_d2d: bad arguments");
  hipEvent_t e0, e1;
  if (int rc = hip_status(hipEventCreate(&e0), "hipEventCreate")) return rc;
  if (int rc = hip_status(hipEventCreate(&e1), "hipEventCreate")) return rc;
  int rc = hip_status(es::launch_copy16(dst, src, bytes, nullptr), "copy warmup");
  if (!rc) rc = hip_status(hipEventRecord(e0, nullptr), "hipEventRecord");
  for (int i = 0; i < reps && !rc; ++i) rc = hip_status(es::launch_copy16(dst, src, bytes, nullptr), "copy");
  if (!rc) rc = hip_status(hipEventRecord(e1, nullptr), "hipEventRecord");
  if (!rc) rc = hip_status(hipEventSynchronize(e1), "hipEventSynchronize");
  float ms = 0.0f;
  if (!rc) rc = hip_status(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (!rc) *ms_avg = ms / reps;
  return rc;
}
int es_synchronize(void) { return hip_status(hipDeviceSynchronize(), "hipDeviceSynchronize"); }
int es_stream_create(void** stream) {
  if (!stream) return fail(ES_ERR_INVALID, "null stream");
  hipStream_t s;
  if (int rc = hip_status(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate"))
    return rc;
  *stream = s;
  return ES_OK;
}
int es_stream_destroy(void* stream) { return hip_status(hipStreamDestroy(S(stream)), "hipStreamDestroy"); }
int es_stream_synchronize(void* stream) {
  return hip_status(hipStreamSynchronize(S(stream)), "hipStreamSynchronize");
}

// ---- LINEAR ----
int es_embedding_q4(const es_q4* table, const uint32_t* token, uint16_t* out, void* stream) {
  es::Q4 t;
  if (!to_q4(table, &t) || t.k != 1024) return fail(ES_ERR_INVALID, "es_embedding_q4: table must be [n,1024] Q4");
  return hip_status(es::launch_embedding(t, token, out, S(stream)), "es_embedding_q4");
}

int es_q4_matvec(const es_q4* w, const uint16_t* x, uint16_t* y, float* y_f32, void* stream) {
  es::Q4 m;
  if (!to_q4(w, &m)) return fail(ES_ERR_INVALID, "es_q4_matvec: null weight");
  return hip_status(es::launch_qmv(m, x, nullptr, y, y_f32, S(stream)), "es_q4_matvec");
}

int es_q4_matvec_add(const es_q4* w, const uint16_t* x, const uint16_t* residual, uint16_t* y,
                     void* stream) {
  es::Q4 m;
  if (!to_q4(w, &m) || !residual) return fail(ES_ERR_INVALID, "es_q4_matvec_add: null argument");
  if (x == y) return fail(ES_ERR_INVALID, "es_q4_matvec_add: x must not alias y");
  return hip_status(es::launch_qmv(m, x, residual, y, nullptr, S(stream)), "es_q4_matvec_add");
}

int es_q4_matvec_rows(const es_q4* w, const uint16_t* x, int rows, const uint16_t* residual, uint16_t* y,
                      void* stream) {
  es::Q4 m;
  if (!to_q4(w, &m) || !x || !y) return fail(ES_ERR_INVALID, "es_q4_matvec_rows: null argument");
  if (rows < 1 || rows > 65535) return fail(ES_ERR_INVALID, "es_q4_matvec_rows: rows must be 1 .. 65535");
  if (x == y) return fail(ES_ERR_INVALID, "es_q4_matvec_rows: x must not alias y");
  return hip_status(es::launch_qmv_rows(m, x, rows, residual, y, nullptr, S(stream)), "es_q4_matvec_rows");
}

int es_linear_row_limit(int n, int k) {
  if (n < 1 || k < 1) return fail(ES_ERR_INVALID, "es_linear_row_limit: n and k must be positive") * -1;
  return es::qmv_row_limit(n, k);
}

int es_add_bf16(const uint16_t* a, const uint16_t* b, int count, uint16_t* out, void* stream) {
  if (!a || !b || !out || count < 1) return fail(ES_ERR_INVALID, "es_add_bf16: null argument or count < 1");
  return hip_status(es::launch_add_bf16(a, b, count, out, S(stream)), "es_add_bf16");
}

int es_greedy_bf16(const uint16_t* logits, int count, void* scratch, size_t scratch_bytes, uint32_t* token,
                   float* lse, void* stream) {
  if (!logits || !token || !scratch) return fail(ES_ERR_INVALID, "es_greedy_bf16: null argument");
  if (count < 1 || count >= (1 << 22)) return fail(ES_ERR_INVALID, "es_greedy_bf16: count must be 1 .. 2^22-1");
  if (scratch_bytes < es::head_scratch_bytes(count))
    return fail(ES_ERR_INVALID, "es_greedy_bf16: scratch smaller than es_head_scratch_bytes(count)");
  return hip_status(es::launch_greedy(logits, count, static_cast<float*>(scratch), token, lse, S(stream)),
                    "es_greedy_bf16");
}

int es_q4_gemm(const es_q4* w, const uint16_t* x, int rows, const uint16_t* residual, uint16_t* y,
               void* stream) {
  es::Q4 m;
  if (!to_q4(w, &m) || !x || !y) return fail(ES_ERR_INVALID, "es_q4_gemm: null argument");
  if (rows < 1 || m.k % 64 != 0) return fail(ES_ERR_INVALID, "es_q4_gemm: rows >= 1 and k % 64 == 0 required");
  if (x == y) return fail(ES_ERR_INVALID, "es_q4_gemm: x must not alias y");
  return hip_status(es::launch_q4_gemm(m, x, rows, residual, y, S(stream)), "es_q4_gemm");
}

int es_q4_gemm_swiglu(const es_q4* gate, const es_q4* up, const uint16_t* x, int rows, uint16_t* act,
                      void* stream) {
  es::Q4 g, u;
  if (!to_q4(gate, &g) || !to_q4(up, &u) || !x || !act) return fail(ES_ERR_INVALID, "es_q4_gemm_swiglu: null argument");
  if (rows < 1 || g.k % 64 != 0 || g.n != u.n || g.k != u.k)
    return fail(ES_ERR_INVALID, "es_q4_gemm_swiglu: rows >= 1, k % 64 == 0 and equal gate/up shapes required");
  if (x == act) return fail(ES_ERR_INVALID, "es_q4_gemm_swiglu: x must not alias act");
  return hip_status(es::launch_q4_gemm_swiglu(g, u, x, rows, act, S(stream)), "es_q4_gemm_swiglu");
}

// ---- prefill row operators ----
int es_embed_rows(const es_q4* embed, const uint32_t* tokens, int rows, uint16_t* h, void* stream) {
  es::Q4 e;
  if (!to_q4(embed, &e) || !tokens || !h) return fail(ES_ERR_INVALID, "es_embed_rows: null argument");
  if (rows < 1 || e.k != 1024) return fail(ES_ERR_INVALID, "es_embed_rows: rows >= 1 and a [vocab, 1024] table required");
  return hip_status(es::launch_embed_rows(e, tokens, rows, h, S(stream)), "es_embed_rows");
}

int es_rmsnorm_rows(const uint16_t* x, const uint16_t* gain, int rows, uint16_t* out, void* stream) {
  if (!x || !gain || !out || rows < 1) return fail(ES_ERR_INVALID, "es_rmsnorm_rows: null argument or rows < 1");
  return hip_status(es::launch_rmsnorm_rows(x, gain, rows, out, S(stream)), "es_rmsnorm_rows");
}

int es_swiglu_rows(const uint16_t* gate, const uint16_t* up, int count, uint16_t* act, void* stream) {
  if (!gate || !up || !act || count < 1) return fail(ES_ERR_INVALID, "es_swiglu_rows: null argument or count < 1");
  return hip_status(es::launch_swiglu_rows(gate, up, count, act, S(stream)), "es_swiglu_rows");
}

int es_gdn_prepare_rows(const uint16_t* raw, uint16_t* ring, const uint16_t* conv_w, const uint16_t* a_proj,
                        const uint16_t* b_proj, const float* a_log, const uint16_t* dt_bias, int position,
                        int rows, uint16_t* q, uint16_t* k, uint16_t* v, float* g, float* beta,
                        void* stream) {
  es::GdnPrepRowsArgs a{raw, ring, conv_w, a_proj, b_proj, a_log, dt_bias, position, rows, q, k, v, g, beta};
  if (!raw || !ring || !conv_w || !a_proj || !b_proj || !a_log || !dt_bias || !q || !k || !v || !g || !beta)
    return fail(ES_ERR_INVALID, "es_gdn_prepare_rows: null argument");
  if (rows < 1 || position < 0) return fail(ES_ERR_INVALID, "es_gdn_prepare_rows: rows >= 1 and position >= 0 required");
  return hip_status(es::launch_gdn_prep_rows(a, S(stream)), "es_gdn_prepare_rows");
}

int es_gdn_recur_rows(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g, const float* beta,
                      int rows, float* state, uint16_t* y, void* stream) {
  if (!q || !k || !v || !g || !beta || !state || !y || rows < 1)
    return fail(ES_ERR_INVALID, "es_gdn_recur_rows: null argument or rows < 1");
  return hip_status(es::launch_gdn_recur_rows(q, k, v, g, beta, rows, state, y, S(stream)), "es_gdn_recur_rows");
}

int es_gdn_conv(const uint16_t* raw, const uint16_t* history, const uint16_t* conv_w, int rows, uint16_t* conv,
                void* stream) {
  if (!raw || !history || !conv_w || !conv) return fail(ES_ERR_INVALID, "es_gdn_conv: null argument");
  if (rows < 1 || rows > (1 << 18)) return fail(ES_ERR_INVALID, "es_gdn_conv: rows must be 1 .. 2^18");
  if (raw == conv) return fail(ES_ERR_INVALID, "es_gdn_conv: raw and conv must be distinct");
  return hip_status(es::launch_gdn_conv_hist(raw, history, conv_w, rows, conv, S(stream)), "es_gdn_conv");
}

int es_gdn_history(const uint16_t* raw, int rows, uint16_t* history, void* stream) {
  if (!raw || !history || rows < 1) return fail(ES_ERR_INVALID, "es_gdn_history: null argument or rows < 1");
  return hip_status(es::launch_gdn_history(raw, rows, history, S(stream)), "es_gdn_history");
}

int es_gdn_prepare(uint16_t* conv, const uint16_t* a_proj, const uint16_t* b_proj, const float* a_log,
                   const uint16_t* dt_bias, int rows, float* g, uint16_t* beta, void* stream) {
  if (!conv || !a_proj || !b_proj || !a_log || !dt_bias || !g || !beta)
    return fail(ES_ERR_INVALID, "es_gdn_prepare: null argument");
  if (rows < 1 || rows > (1 << 24)) return fail(ES_ERR_INVALID, "es_gdn_prepare: rows must be 1 .. 2^24");
  return hip_status(es::launch_gdn_prepare_hist(conv, a_proj, b_proj, a_log, dt_bias, rows, g, beta, S(stream)),
                    "es_gdn_prepare");
}

int es_gdn_recur(const uint16_t* conv, const float* g, const uint16_t* beta, int rows, float* state, uint16_t* y,
                 void* stream) {
  if (!conv || !g || !beta || !state || !y || rows < 1) return fail(ES_ERR_INVALID, "es_gdn_recur: null argument or rows < 1");
  return hip_status(es::launch_gdn_recur_conv(conv, g, beta, rows, state, y, S(stream)), "es_gdn_recur");
}

int es_gdn_norm_gate_rows(const uint16_t* y, const uint16_t* z, const uint16_t* norm_w, int rows, uint16_t* out,
                          void* stream) {
  if (!y || !z || !norm_w || !out || rows < 1) return fail(ES_ERR_INVALID, "es_gdn_norm_gate_rows: null argument or rows < 1");
  return hip_status(es::launch_gdn_norm_gate_rows(y, z, norm_w, rows, out, S(stream)), "es_gdn_norm_gate_rows");
}

int es_attn_prepare_rows(const uint16_t* q_proj, const uint16_t* k_proj, const uint16_t* v_proj,
                         const uint16_t* q_gain, const uint16_t* k_gain, const float* inv_freq, int position,
                         int rows, uint16_t* query, uint16_t* kcache, uint16_t* vcache, int capacity,
                         void* stream) {
  es::AttnPrepRowsArgs a{q_proj, k_proj, v_proj, q_gain, k_gain, inv_freq, position, rows, query, kcache, vcache,
                         capacity};
  if (!q_proj || !k_proj || !v_proj || !q_gain || !k_gain || !inv_freq || !query || !kcache || !vcache)
    return fail(ES_ERR_INVALID, "es_attn_prepare_rows: null argument");
  if (rows < 1 || position < 0 || (int64_t)position + rows > capacity)
    return fail(ES_ERR_INVALID, "es_attn_prepare_rows: rows >= 1 and 0 <= position, position + rows <= capacity required");
  return hip_status(es::launch_attn_prep_rows(a, S(stream)), "es_attn_prepare_rows");
}

int es_attn_prefill(const uint16_t* query, const uint16_t* kcache, const uint16_t* vcache, int position, int rows,
                    int capacity, uint16_t* out, void* stream) {
  if (!query || !kcache || !vcache || !out) return fail(ES_ERR_INVALID, "es_attn_prefill: null argument");
  if (rows < 1 || position < 0 || (int64_t)position + rows > capacity)
    return fail(ES_ERR_INVALID, "es_attn_prefill: rows >= 1 and 0 <= position, position + rows <= capacity required");
  return hip_status(es::launch_attn_prefill(query, kcache, vcache, position, rows, capacity, out, S(stream)),
                    "es_attn_prefill");
}

int es_attn_gate_rows(const uint16_t* o, const uint16_t* q_proj, int rows, uint16_t* gated, void* stream) {
  if (!o || !q_proj || !gated || rows < 1) return fail(ES_ERR_INVALID, "es_attn_gate_rows: null argument or rows < 1");
  return hip_status(es::launch_attn_gate_rows(o, q_proj, rows, gated, S(stream)), "es_attn_gate_rows");
}

int es_q4_rmsnorm_matvec_multi(const es_q4* w, int count, const uint16_t* x, const uint16_t* gain,
                               uint16_t* norm_out, uint16_t* const* y, void* stream) {
  if (count < 1 || count > 4 || !w || !y || !x) return fail(ES_ERR_INVALID, "es_q4_rmsnorm_matvec_multi: bad count/pointers");
  es::NormMultiArgs a{};
  a.count = count;
  for (int i = 0; i < count; ++i) {
    if (!to_q4(&w[i], &a.m[i])) return fail(ES_ERR_INVALID, "es_q4_rmsnorm_matvec_multi: null weight");
    a.y[i] = y[i];
  }
  a.x = x;
  a.gain = gain;
  a.norm_out = norm_out;
  return hip_status(es::launch_norm_multi(a, S(stream)), "es_q4_rmsnorm_matvec_multi");
}

int es_q4_rmsnorm_gate_up_swiglu(const es_q4* gate, const es_q4* up, const uint16_t* x,
                                 const uint16_t* gain, uint16_t* norm_out, uint16_t* act,
                                 void* stream) {
  es::Q4 g, u;
  if (!to_q4(gate, &g) || !to_q4(up, &u)) return fail(ES_ERR_INVALID, "es_q4_rmsnorm_gate_up_swiglu: null weight");
  return hip_status(es::launch_norm_gate_up(g, u, x, gain, norm_out, act, S(stream)),
                    "es_q4_rmsnorm_gate_up_swiglu");
}

// ---- GDN ----
int es_gdn_in_proj(const es_q4* qkv, const es_q4* z, const es_q4* a, const es_q4* b,
                   const uint16_t* x, const uint16_t* gain, uint16_t* norm_out, uint16_t* ring,
                   int position, uint16_t* z_out, uint16_t* ab_out, void* stream) {
  es::NormMultiArgs n{};
  n.count = 4;
  if (!to_q4(qkv, &n.m[0]) || !to_q4(z, &n.m[1]) || !to_q4(a, &n.m[2]) || !to_q4(b, &n.m[3]))
    return fail(ES_ERR_INVALID, "es_gdn_in_proj: null weight");
  if (n.m[0].n != 6144 || n.m[1].n != 2048 || n.m[2].n != 16 || n.m[3].n != 16)
    return fail(ES_ERR_INVALID, "es_gdn_in_proj: expected qkv 6144, z 2048, a 16, b 16 rows");
  if (position < 0 || !ring || !z_out || !ab_out) return fail(ES_ERR_INVALID, "es_gdn_in_proj: bad position/pointers");
  n.y[0] = ring;
  n.y[1] = z_out;
  n.y[2] = ab_out;
  n.y[3] = ab_out + 16;
  n.ring0 = 1;
  n.pos_val = position;
  n.x = x;
  n.gain = gain;
  n.norm_out = norm_out;
  return hip_status(es::launch_norm_multi(n, S(stream)), "es_gdn_in_proj");
}

int es_gdn_recur_step(const uint16_t* ring, int position, const uint16_t* conv_w,
                      const uint16_t* ab, const float* a_log, const uint16_t* dt_bias,
                      float* state, uint16_t* y, uint16_t* qkv_out, float* g_out,
                      uint16_t* beta_out, void* stream) {
  if (position < 0) return fail(ES_ERR_INVALID, "es_gdn_recur_step: negative position");
  es::GdnRecurArgs g{};
  g.ring = ring;
  g.conv_w = conv_w;
  g.ab = ab;
  g.a_log = a_log;
  g.dt_bias = dt_bias;
  g.state = state;
  g.y = y;
  g.qkv_out = qkv_out;
  g.g_out = g_out;
  g.beta_out = beta_out;
  g.pos_val = position;
  return hip_status(es::launch_gdn_recur(g, S(stream)), "es_gdn_recur_step");
}

int es_gdn_gate_out_proj(const es_q4* out_proj, const uint16_t* y, const uint16_t* z,
                         const uint16_t* norm_w, uint16_t* h, uint16_t* gated_out, void* stream) {
  es::Q4 m;
  if (!to_q4(out_proj, &m)) return fail(ES_ERR_INVALID, "es_gdn_gate_out_proj: null weight");
  return hip_status(es::launch_gdn_gate_out(m, y, z, norm_w, h, gated_out, S(stream)),
                    "es_gdn_gate_out_proj");
}

// ---- attention ----
int es_rope_inv_freq(float* host_out32) {
  if (!host_out32) return fail(ES_ERR_INVALID, "null output");
  for (int i = 0; i < 32; ++i) host_out32[i] = es::rope_inv_freq_host(i);
  return ES_OK;
}

size_t es_attn_scratch_bytes(int capacity) {
  if (capacity < 1) return 0;
  return es::attn_scratch_bytes(capacity);
}

int es_attn_decode(const uint16_t* q_proj, const uint16_t* k_proj, const uint16_t* v_proj,
                   const uint16_t* q_gain, const uint16_t* k_gain, uint16_t* kcache,
                   uint16_t* vcache, int capacity, int position, const float* inv_freq,
                   int blocks, void* scratch, size_t scratch_bytes, uint16_t* gated,
                   uint16_t* query_out, void* stream) {
  if (blocks < 1 || blocks > 1024) return fail(ES_ERR_INVALID, "es_attn_decode: blocks must be 1..1024");
  if (position < 0 || position >= capacity) return fail(ES_ERR_INVALID, "es_attn_decode: position outside capacity");
  if (!scratch || scratch_bytes < es::attn_scratch_bytes(capacity))
    return fail(ES_ERR_INVALID, "es_attn_decode: scratch too small");
  es::AttnArgs a{};
  a.q_proj = q_proj;
  a.k_proj = k_proj;
  a.v_proj = v_proj;
  a.q_gain = q_gain;
  a.k_gain = k_gain;
  a.kcache = kcache;
  a.vcache = vcache;
  a.capacity = capacity;
  a.inv_freq = inv_freq;
  es::attn_bind_scratch(a, scratch);
  a.blocks = blocks;
  a.gated = gated;
  a.query_out = query_out;
  a.pos_val = position;
  if (int rc = hip_status(es::launch_attn_fused(a, S(stream)), "es_attn_decode chains")) return rc;
  return hip_status(es::launch_attn_merge(a, S(stream)), "es_attn_decode merge");
}

// ---- head ----
size_t es_head_scratch_bytes(int vocab) {
  if (vocab < 1) return 0;
  return es::head_scratch_bytes(vocab);
}

int es_head_greedy(const es_q4* embed, const uint16_t* h, const uint16_t* gain,
                   uint16_t* norm_out, uint16_t* logits, void* scratch, size_t scratch_bytes,
                   uint32_t* token, float* lse, void* stream) {
  es::HeadArgs a{};
  if (!to_q4(embed, &a.embed) || a.embed.k != 1024) return fail(ES_ERR_INVALID, "es_head_greedy: table must be [vocab,1024] Q4");
  if (!scratch || scratch_bytes < es::head_scratch_bytes(a.embed.n))
    return fail(ES_ERR_INVALID, "es_head_greedy: scratch too small");
  a.h = h;
  a.gain = gain;
  a.norm_out = norm_out;
  a.logits = logits;
  a.part = static_cast<float*>(scratch);
  a.token_out = token;
  a.lse_out = lse;
  return hip_status(es::launch_head(a, S(stream)), "es_head_greedy");
}

int es_head_greedy_noalloc(const es_q4* embed, const uint16_t* h, const uint16_t* gain, uint16_t* norm_out,
                           uint16_t* logits, uint32_t* token, float* lse, void* stream) {
  es::HeadArgs a{};
  if (!to_q4(embed, &a.embed) || a.embed.k != 1024)
    return fail(ES_ERR_INVALID, "es_head_greedy_noalloc: table must be [vocab,1024] Q4");
  if (a.embed.n > ES_HEAD_NOALLOC_MAX_VOCAB || a.embed.n > es::head_noalloc_max_vocab())
    return fail(ES_ERR_INVALID, "es_head_greedy_noalloc: vocab " + std::to_string(a.embed.n) +
                                    " exceeds the in-library scratch limit of " +
                                    std::to_string(ES_HEAD_NOALLOC_MAX_VOCAB) + " rows");
  if (!h || !gain || !logits || !token) return fail(ES_ERR_INVALID, "es_head_greedy_noalloc: null argument");
  a.h = h;
  a.gain = gain;
  a.norm_out = norm_out;
  a.logits = logits;
  a.token_out = token;
  a.lse_out = lse;
  return hip_status(es::launch_head_noalloc(a, S(stream)), "es_head_greedy_noalloc");
}

// ---- weights ----
size_t es_weights_total_bytes(int n_layers, int vocab) {
  if (n_layers < 1 || vocab < 1) return 0;
  uint64_t total = 0;
  es::weight_layout({n_layers, vocab}, &total);
  return total;
}

int es_weights_tensor_count(int n_layers) {
  if (n_layers < 1) return 0;
  return (int)es::weight_layout({n_layers, 1}, nullptr).size();
}

int es_weights_tensor_info(int n_layers, int vocab, int index, char* name, int name_len,
                           uint64_t* offset, uint64_t* bytes, int* dtype) {
  if (n_layers < 1 || vocab < 1) return fail(ES_ERR_INVALID, "bad model shape");
  const auto t = es::weight_layout({n_layers, vocab}, nullptr);
  if (index < 0 || index >= (int)t.size()) return fail(ES_ERR_INVALID, "tensor index out of range");
  if (name && name_len > 0) {
    std::strncpy(name, t[index].name.c_str(), name_len - 1);
    name[name_len - 1] = 0;
  }
  if (offset) *offset = t[index].offset;
  if (bytes) *bytes = t[index].bytes;
  if (dtype) *dtype = (int)t[index].dtype;
  return ES_OK;
}

int es_weights_tensor_shape(int n_layers, int vocab, int index, int64_t* dims, int max_dims) {
  if (n_layers < 1 || vocab < 1) return fail(ES_ERR_INVALID, "bad model shape");
  const auto t = es::weight_layout({n_layers, vocab}, nullptr);
  if (index < 0 || index >= (int)t.size()) return fail(ES_ERR_INVALID, "tensor index out of range");
  const int nd = (int)t[index].shape.size();
  if (!dims || max_dims < nd) return fail(ES_ERR_INVALID, "es_weights_tensor_shape: dims too short");
  for (int i = 0; i < nd; ++i) dims[i] = t[index].shape[i];
  return nd;
}

int es_weights_random(int n_layers, int vocab, uint64_t seed, void* blob, size_t bytes,
                      int threads) {
  if (n_layers < 1 || vocab < 1) return fail(ES_ERR_INVALID, "bad model shape");
  if (!es::weights_random({n_layers, vocab}, seed, blob, bytes, threads))
    return fail(ES_ERR_INVALID, "es_weights_random: blob too small");
  return ES_OK;
}

int es_checkpoint_config(const char* model_dir, int* n_layers, int* vocab) {
  if (!model_dir || !n_layers || !vocab) return fail(ES_ERR_INVALID, "es_checkpoint_config: null argument");
  std::string err;
  if (!es::checkpoint_config(model_dir, n_layers, vocab, &err)) return fail(ES_ERR_INVALID, err);
  return ES_OK;
}

int es_checkpoint_load(const char* model_dir, int n_layers, int vocab, void* blob, size_t bytes) {
  if (!model_dir || n_layers < 1 || vocab < 1) return fail(ES_ERR_INVALID, "es_checkpoint_load: bad arguments");
  std::string err;
  if (!es::checkpoint_load(model_dir, n_layers, vocab, blob, bytes, &err)) return fail(ES_ERR_INVALID, err);
  return ES_OK;
}

// ---- engine ----
es_engine* es_engine_create(const void* blob, size_t bytes, int n_layers, int vocab,
                            int capacity) {
  std::string err;
  es::Engine* e = es::Engine::create(blob, bytes, n_layers, vocab, capacity, &err);
  if (!e) {
    fail(ES_ERR_INVALID, err);
    return nullptr;
  }
  return new es_engine{e};
}

void es_engine_destroy(es_engine* e) {
  if (!e) return;
  delete e->impl;
  delete e;
}

int es_engine_generate(es_engine* e, const uint32_t* prompt, int len, int max_tokens, int reset,
                       uint32_t* out) {
  if (!e || !out) return fail(ES_ERR_INVALID, "null engine/output");
  std::string err;
  return engine_rc(e->impl->generate(prompt, len, max_tokens, reset != 0, out, &err), err);
}

int es_engine_set_prefill(es_engine* e, int chunk_rows) {
  if (!e) return fail(ES_ERR_INVALID, "null engine");
  std::string err;
  return engine_rc(e->impl->set_prefill(chunk_rows, &err), err);
}

int es_engine_xcd_kernels(const es_engine* e) {
  if (!e || !e->impl) return fail(ES_ERR_INVALID, "es_engine_xcd_kernels: null engine") * -1;
  return e->impl->fused_mlp() ? 1 : 0;
}

int es_engine_set_xcd_kernels(es_engine* e, int on) {
  if (!e || !e->impl) return fail(ES_ERR_INVALID, "null engine");
  std::string err;
  return engine_rc(e->impl->set_xcd_kernels(on != 0, &err), err);
}

int es_engine_inject_exchange_fault(es_engine* e, int mode) {
  if (!e || !e->impl) return fail(ES_ERR_INVALID, "null engine");
  std::string err;
  return engine_rc(e->impl->inject_exchange_fault(mode, &err), err);
}

int es_engine_prompt_split(const es_engine* e, int* chunks, int* routed_rows, int* decode_rows) {
  if (!e || !e->impl || !chunks || !routed_rows || !decode_rows)
    return fail(ES_ERR_INVALID, "es_engine_prompt_split: null argument");
  const es::Engine::PromptSplit p = e->impl->last_prompt_split();
  *chunks = p.chunks;
  *routed_rows = p.routed_rows;
  *decode_rows = p.decode_rows;
  return ES_OK;
}

void es_engine_cancel(es_engine* e) {
  if (e) e->impl->cancel();
}
void es_engine_clear_cancel(es_engine* e) {
  if (e) e->impl->clear_cancel();
}
int es_engine_position(const es_engine* e) { return e ? e->impl->position() : -1; }

int es_engine_forced_decode(es_engine* e, const uint32_t* tokens, int n, uint32_t* argmax,
                            uint16_t* logits) {
  if (!e) return fail(ES_ERR_INVALID, "null engine");
  std::string err;
  return engine_rc(e->impl->forced_decode(tokens, n, argmax, logits, &err), err);
}

int es_engine_read_kv(es_engine* e, int layer, int which, int pos0, int count, void* host) {
  if (!e) return fail(ES_ERR_INVALID, "null engine");
  std::string err;
  return engine_rc(e->impl->read_kv(layer, which, pos0, count, host, &err), err);
}
int es_engine_write_kv(es_engine* e, int layer, int which, int pos0, int count,
                       const void* host) {
  if (!e) return fail(ES_ERR_INVALID, "null engine");
  std::string err;
  return engine_rc(e->impl->write_kv(layer, which, pos0, count, host, &err), err);
}
int es_engine_read_gdn(es_engine* e, int layer, void* ring, void* state) {
  if (!e) return fail(ES_ERR_INVALID, "null engine");
  std::string err;
  return engine_rc(e->impl->read_gdn(layer, ring, state, &err), err);
}
int es_engine_write_gdn(es_engine* e, int layer, const void* ring, const void* state) {
  if (!e) return fail(ES_ERR_INVALID, "null engine");
  std::string err;
  return engine_rc(e->impl->write_gdn(layer, ring, state, &err), err);
}
int es_engine_set_position(es_engine* e, int position, uint32_t pending) {
  if (!e) return fail(ES_ERR_INVALID, "null engine");
  std::string err;
  return engine_rc(e->impl->set_position(position, pending, &err), err);
}
int es_engine_fill_synthetic(es_engine* e, int length, uint64_t seed, uint32_t pending) {
  if (!e) return fail(ES_ERR_INVALID, "null engine");
  std::string err;
  return engine_rc(e->impl->fill_synthetic(length, seed, pending, &err), err);
}
int es_engine_time_decode(es_engine* e, int steps, int warmup, double* ms_total) {
  if (!e || !ms_total) return fail(ES_ERR_INVALID, "null engine/output");
  std::string err;
  return engine_rc(e->impl->time_decode(steps, warmup, ms_total, &err), err);
}
int es_engine_time_attention(es_engine* e, int layer, int reps, int which, double* ms_avg) {
  if (!e || !ms_avg) return fail(ES_ERR_INVALID, "null engine/output");
  std::string err;
  return engine_rc(e->impl->time_attention(layer, reps, which, ms_avg, &err), err);
}
int es_engine_time_head(es_engine* e, int reps, double* ms_avg) {
  if (!e || !ms_avg) return fail(ES_ERR_INVALID, "null engine/output");
  std::string err;
  return engine_rc(e->impl->time_head(reps, ms_avg, &err), err);
}
int es_engine_splits_for(int length) { return es::Engine::splits_for(length); }

}  // extern "C"
