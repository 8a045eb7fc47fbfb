/*
 * es_decode.h -- C ABI of the MI355X decode engine (libesdecode.so).
 *
 * Two boundaries of the reference are kept:
 *  1. the kernel/operator boundary: the LINEAR, GDN and ATTENTION kernel
 *     interfaces (source/LINEAR_INTERFACE.md, source/GDN_INTERFACE.md,
 *     source/ATTENTION_INTERFACE.md) that the reference reaches through
 *     Gpu::dispatch (source/src/gpu.rs:69-80);
 *  2. the engine boundary: Model::load / Model::generate / cancelled
 *     (source/src/model.rs:28-122), which the EngineSmith protocol server
 *     (source/src/main.rs:10-53, docs/protocol.md) drives.
 *
 * Conventions (as in the reference): tensors are positional, row-major, bf16
 * values are raw uint16_t, Q4 weights are the MLX affine 4-bit group-64
 * triple. Operator pointers are DEVICE pointers owned by the caller; no
 * operator allocates. `stream` is a hipStream_t (NULL = default stream); ops
 * are asynchronous on it. Every function returns 0 (ES_OK) or an error code,
 * with a message from es_last_error() (thread-local). Launch failures are
 * reported when detected; asynchronous device faults surface at the next
 * synchronising call, as Gpu::wait reports them (gpu.rs:61-64).
 * An engine instance is not thread-safe, except es_engine_cancel.
 */
#ifndef ES_DECODE_H
#define ES_DECODE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ES_OK 0
#define ES_ERR_INVALID 1   /* bad argument or request (reference `ensure!`) */
#define ES_ERR_DEVICE 2    /* HIP runtime / launch failure */
#define ES_ERR_CANCELLED 3 /* input disconnected (model.rs:133) */

/* Text of the last error on this thread ("" if none). */
const char* es_last_error(void);

/* Q4 affine group-64 weight: codes u32 [n, k/8] (nibble j of word w is column
 * 8w+j), bf16 scales and biases [n, k/64]. Replaces `Linear` (weights.rs:8,
 * 50-52). */
typedef struct es_q4 {
  const uint32_t* codes;
  const uint16_t* scales;
  const uint16_t* biases;
  int32_t n;
  int32_t k;
} es_q4;

/* ------------------------------------------------------------------ */
/* Device plumbing (stands in for Gpu::new/buffer/zero/finish,         */
/* gpu.rs:18-68)                                                       */
/* ------------------------------------------------------------------ */
int es_device_count(int* count);
int es_device_name(int device, char* buf, int len);
int es_set_device(int device);
int es_malloc(void** ptr, size_t bytes);
int es_free(void* ptr);
int es_memcpy_htod(void* dst, const void* src, size_t bytes);
int es_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int es_memset(void* dst, int value, size_t bytes);
/* Device-to-device copy by a plain streaming kernel (bytes a multiple of
 * 16); no reference counterpart: plumbing, and the known-size workload that
 * calibrates the HBM byte counters. */
int es_copy_d2d(void* dst, const void* src, size_t bytes, void* stream);
/* Average ms of `reps` es_copy_d2d launches on the null stream (HIP events):
 * the measured streaming-copy peak beside the nameplate HBM figure. */
int es_time_copy_d2d(void* dst, const void* src, size_t bytes, int reps, double* ms_avg);
/* Average ms of `reps` launches of a plain streaming-read kernel over `bytes`
 * (a multiple of 2 MiB) at src: 256 blocks, each reading a contiguous chunk
 * by 16-byte global->LDS DMA, the fastest read pattern measured on MI355X;
 * out is device scratch of at least 1 KiB. No reference counterpart: the
 * measured read-only ceiling beside the nameplate HBM figure, for kernels
 * that only read. */
int es_time_read(const void* src, size_t bytes, void* out, size_t out_bytes, int reps, double* ms_avg);
int es_synchronize(void);
int es_stream_create(void** stream);
int es_stream_destroy(void* stream);
int es_stream_synchronize(void* stream);

/* ------------------------------------------------------------------ */
/* LINEAR interface (LINEAR_INTERFACE.md:16-25)                        */
/* ------------------------------------------------------------------ */
/* embedding_q4 (linear.metal:11-24): out[1024] = bf16(scale*q + bias) of
 * row *token (token is a device pointer, as the reference's ids buffer). */
int es_embedding_q4(const es_q4* table, const uint32_t* token, uint16_t* out, void* stream);

/* qmv_q4 (linear.metal:28-73), M=1: y[n] = bf16(W x). k == 1024, or
 * 1024 < k <= 4096 with k % 64 == 0. y_f32 (optional) gets the fp32 sums. */
int es_q4_matvec(const es_q4* w, const uint16_t* x, uint16_t* y, float* y_f32, void* stream);

/* qmv_add_q4 (linear.metal:77-123): y = bf16(residual + bf16(W x)).
 * y may alias residual; x must not alias y (LINEAR_INTERFACE.md:35-36). */
int es_q4_matvec_add(const es_q4* w, const uint16_t* x, const uint16_t* residual, uint16_t* y,
                     void* stream);

/* qmv_q4 with M = rows token rows (LINEAR_INTERFACE.md:19; linear.metal:28-73):
 * y[r] = bf16(W x[r]), or with residual (may alias y) bf16(residual[r] +
 * bf16(W x[r])). x [rows, k], y and residual [rows, n]; each row has the
 * M = 1 arithmetic of es_q4_matvec. k as for es_q4_matvec; rows 1 .. 65535;
 * x must not alias y. */
int es_q4_matvec_rows(const es_q4* w, const uint16_t* x, int rows, const uint16_t* residual, uint16_t* y,
                      void* stream);

/* Row count from which the reference's batched linear of an [n, k] matrix
 * leaves qmv_q4 for the GEMM (Model::linear, model.rs:189-192): 33 when
 * k <= 2048 and n <= 2048, else 25 when k <= 4096 and n <= 4096, else 13.
 * A forward of fewer rows runs that linear as es_q4_matvec_rows. Returns
 * -ES_ERR_INVALID for non-positive shapes. */
int es_linear_row_limit(int n, int k);

/* add_bf16 (LINEAR_INTERFACE.md:23; linear.metal:372-379): out[i] =
 * bf16(a[i] + b[i]) for count elements; out may alias a or b. */
int es_add_bf16(const uint16_t* a, const uint16_t* b, int count, uint16_t* out, void* stream);

/* greedy_bf16 (LINEAR_INTERFACE.md:25,38-42; linear.metal:400-449) over bf16
 * logits[count]: lse = bf16(log(sum exp) + max), *token = lowest index of the
 * maximum of bf16(logit - lse), in the order es_head_greedy uses (token and
 * lse are device pointers; lse optional). scratch: es_head_scratch_bytes(count)
 * bytes of device memory. count 1 .. 2^22-1. */
int es_greedy_bf16(const uint16_t* logits, int count, void* scratch, size_t scratch_bytes, uint32_t* token,
                   float* lse, void* stream);

/* Row-batched LINEAR (prefill, rows > 1; model.rs:189-199 routes it to
 * qmm_q4_nax, linear_nax.metal:1096-1139): y[r,n] = bf16(sum_k x[r,k] *
 * bf16(scale*q + bias)) with fp32 accumulation, or with residual (may alias
 * y) bf16(residual[r,n] + that). x is [rows, k], y [rows, n]; k % 64 == 0;
 * x must not alias y. */
int es_q4_gemm(const es_q4* w, const uint16_t* x, int rows, const uint16_t* residual, uint16_t* y,
               void* stream);

/* The MLP's row-batched gate and up linears and swiglu_bf16 (model.rs:
 * 279-282; linear.metal:382-398) in one GEMM: act [rows, n] =
 * bf16(bf16(g * sigmoid(g)) * u) with g, u the bf16 outputs es_q4_gemm gives
 * for gate and up; bitwise the same as those three operators. */
int es_q4_gemm_swiglu(const es_q4* gate, const es_q4* up, const uint16_t* x, int rows, uint16_t* act,
                      void* stream);

/* ------------------------------------------------------------------ */
/* Prefill row operators (encode_forward with rows > 1, model.rs:228-343) */
/* ------------------------------------------------------------------ */
/* Each reproduces its decode counterpart's arithmetic row by row; rows are
 * consecutive tokens at positions position .. position+rows-1. */

/* embedding_q4 (linear.metal:11-24): h [rows, 1024] = bf16(scale*q + bias) of
 * each token's table row. Tokens outside the table read row 0. */
int es_embed_rows(const es_q4* embed, const uint32_t* tokens, int rows, uint16_t* h, void* stream);

/* rms_norm_bf16 (linear.metal:300-333, eps 1e-6): out [rows, 1024]. */
int es_rmsnorm_rows(const uint16_t* x, const uint16_t* gain, int rows, uint16_t* out, void* stream);

/* swiglu_bf16 (linear.metal:382-398) over `count` elements:
 * act = bf16(bf16(gate*sigmoid(gate)) * up). */
int es_swiglu_rows(const uint16_t* gate, const uint16_t* up, int count, uint16_t* act, void* stream);

/* gdn_conv + gdn_history + gdn_prepare (gdn.metal:33-120): raw [rows, 6144]
 * projected q|k|v; ring [4, 6144] holds the raw rows of earlier positions in
 * slot (position & 3) and receives the chunk's last min(rows, 4) rows;
 * a_proj, b_proj [rows, 16]. Outputs q, k [rows, 16, 128] (L2-normalised and
 * scaled), v [rows, 16, 128] (SiLU of the convolution), g, beta [rows, 16]
 * fp32. */
int es_gdn_prepare_rows(const uint16_t* raw, uint16_t* ring, const uint16_t* conv_w, const uint16_t* a_proj,
                        const uint16_t* b_proj, const float* a_log, const uint16_t* dt_bias, int position,
                        int rows, uint16_t* q, uint16_t* k, uint16_t* v, float* g, float* beta,
                        void* stream);

/* gdn_recur with rows > 1 (gdn.metal:176-228): the delta-rule update of state
 * [16, 128v, 128k] fp32 (in place) for each row in order; y [rows, 2048]. */
int es_gdn_recur_rows(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g, const float* beta,
                      int rows, float* state, uint16_t* y, void* stream);

/* The reference's GDN kernels over its history form (GDN_INTERFACE.md:8-18):
 * history [3, 6144] bf16, oldest row first, zero after a reset; row-major
 * [rows, ...] tensors with tokens outer. Call in the order gdn_conv,
 * gdn_history, gdn_prepare, gdn_recur, gdn_norm_gate (es_gdn_norm_gate_rows)
 * on one stream. Arithmetic as the decode step's (es_gdn_recur_step). */

/* gdn_conv (gdn.metal:31-51): conv [rows, 6144] = bf16(x * sigmoid_bf(x)),
 * x = bf16(four-tap fma chain over the raw rows, taps before row 0 from the
 * history). raw and conv must be distinct; rows 1 .. 2^18. */
int es_gdn_conv(const uint16_t* raw, const uint16_t* history, const uint16_t* conv_w, int rows, uint16_t* conv,
                void* stream);
/* gdn_history (gdn.metal:53-73): history (in place) takes the last three raw
 * rows; with rows < 3 its newest rows shift down. Run after es_gdn_conv. */
int es_gdn_history(const uint16_t* raw, int rows, uint16_t* history, void* stream);
/* gdn_prepare (gdn.metal:75-114): q and k of each head normalised in place in
 * conv (bf16(bf16(x * rsqrt(mean(x^2) + 1e-6/128)) * scale), scale 1/128 for
 * q, bf16(128^-1/2) for k); g [rows,16] fp32 = exp(-exp(A_log) *
 * softplus(bf16(a + dt_bias))), beta [rows,16] bf16 = sigmoid_bf(b). */
int es_gdn_prepare(uint16_t* conv, const uint16_t* a_proj, const uint16_t* b_proj, const float* a_log,
                   const uint16_t* dt_bias, int rows, float* g, uint16_t* beta, void* stream);
/* gdn_recur (gdn.metal:176-228) over the normalised conv buffer [rows, 6144]
 * (q | k | v blocks of 2048): the delta-rule update of state [16,128v,128k]
 * fp32 (in place) for each row in order; y [rows, 2048] bf16. */
int es_gdn_recur(const uint16_t* conv, const float* g, const uint16_t* beta, int rows, float* state, uint16_t* y,
                 void* stream);

/* gdn_norm_gate (gdn.metal:230-255): out [rows, 2048] =
 * bf16(SiLU(z) * bf16(bf16(y * rsqrt(mean(y^2) + 1e-6)) * norm_w)) per head. */
int es_gdn_norm_gate_rows(const uint16_t* y, const uint16_t* z, const uint16_t* norm_w, int rows, uint16_t* out,
                          void* stream);

/* attn_prepare_q + attn_prepare_kv (attention.metal:72-131): per row, query
 * [rows, 8, 256] = RoPE(RMSNorm(q head) * q_gain) at its position; K row =
 * RoPE(RMSNorm(k head) * k_gain) and V row written to kcache/vcache
 * [2, capacity, 256] at that position. q_proj [rows, 8, 512] (query|gate). */
int es_attn_prepare_rows(const uint16_t* q_proj, const uint16_t* k_proj, const uint16_t* v_proj,
                         const uint16_t* q_gain, const uint16_t* k_gain, const float* inv_freq, int position,
                         int rows, uint16_t* query, uint16_t* kcache, uint16_t* vcache, int capacity,
                         void* stream);

/* attn_prefill (attention_prefill.metal:2256; model.rs:337-343): causal GQA
 * attention, row r attends to cache positions 0 .. position+r; out
 * [rows, 8, 256] = bf16(softmax(q.K^T / 16) V), fp32 softmax, products on
 * bf16 operands (the probabilities rounded to bf16) with fp32 accumulation.
 * capacity is at most 2^22 rows. */
int es_attn_prefill(const uint16_t* query, const uint16_t* kcache, const uint16_t* vcache, int position, int rows,
                    int capacity, uint16_t* out, void* stream);

/* attn_gate (attention.metal:133-151): gated [rows, 2048] =
 * bf16(o * sigmoid(gate)), gate the second half of each q_proj head. */
int es_attn_gate_rows(const uint16_t* o, const uint16_t* q_proj, int rows, uint16_t* gated, void* stream);

/* qmv_multi_g8_norm (linear_input_norm.metal:13-119) with the rms_norm_bf16
 * arithmetic (linear.metal:300-331): u = bf16(bf16(x*rsqrt(mean(x^2)+1e-6))*gain)
 * over 1024 columns, then y[i] = bf16(W_i u) for count (1..4) matrices of
 * k = 1024, each with a multiple of 8 rows. norm_out (optional) receives u. */
int es_q4_rmsnorm_matvec_multi(const es_q4* w, int count, const uint16_t* x, const uint16_t* gain,
                               uint16_t* norm_out, uint16_t* const* y, void* stream);

/* qmv_mlp_g8_norm (linear_norm.metal:10-104): u = RMSNorm(x)*gain, then
 * act = bf16(bf16(g*sigmoid_bf(g)) * up) with g = bf16(Wg u), up = bf16(Wu u). */
int es_q4_rmsnorm_gate_up_swiglu(const es_q4* gate, const es_q4* up, const uint16_t* x,
                                 const uint16_t* gain, uint16_t* norm_out, uint16_t* act,
                                 void* stream);

/* ------------------------------------------------------------------ */
/* GDN interface (GDN_INTERFACE.md:12-18; decode fusion gdn_input.metal) */
/* ------------------------------------------------------------------ */
/* Convolution history is kept as a ring of the last four raw qkv projections,
 * ring [4, 6144] bf16, slot = position & 3. The reference's history [3, 6144]
 * (oldest first) maps to ring slots (position-3)&3, (position-2)&3,
 * (position-1)&3; nothing is shifted. A reset ring is all zeros, as the
 * reference's reset history (model.rs:95). */

/* Projection half of gdn_input_g16 (gdn_input.metal:109-155): u = RMSNorm(x)*gain
 * (1024), raw qkv = W_qkv u written to ring slot (position & 3), z = W_z u
 * [2048], ab = [W_a u (16) | W_b u (16)]. */
int es_gdn_in_proj(const es_q4* qkv, const es_q4* z, const es_q4* a, const es_q4* b,
                   const uint16_t* x, const uint16_t* gain, uint16_t* norm_out, uint16_t* ring,
                   int position, uint16_t* z_out, uint16_t* ab_out, void* stream);

/* Convolution/preparation half of gdn_input_g16 (gdn_input.metal:157-205,
 * == gdn_conv_prepare_decode, gdn.metal:121-171) fused with gdn_recur
 * (gdn.metal:176-228), T=1: conv over ring slots position-3..position, SiLU,
 * Q/K L2 norm, g/beta gates, delta-rule update of state [16,128v,128k] fp32 in
 * place, y [2048] bf16. Optional debug outputs: qkv_out [6144] (normalised
 * q|k, activated v), g_out [16] fp32, beta_out [16] bf16. */
int es_gdn_recur_step(const uint16_t* ring, int position, const uint16_t* conv_w,
                      const uint16_t* ab, const float* a_log, const uint16_t* dt_bias,
                      float* state, uint16_t* y, uint16_t* qkv_out, float* g_out,
                      uint16_t* beta_out, void* stream);

/* gdn_norm_gate (gdn.metal:230-255) feeding out_proj with the residual
 * (qmv_add_q4, model.rs:265): h = bf16(h + bf16(W_out gated)) in place.
 * gated_out (optional) receives the gated vector [2048]. */
int es_gdn_gate_out_proj(const es_q4* out_proj, const uint16_t* y, const uint16_t* z,
                         const uint16_t* norm_w, uint16_t* h, uint16_t* gated_out, void* stream);

/* ------------------------------------------------------------------ */
/* ATTENTION interface (ATTENTION_INTERFACE.md:13-29, 75-105)          */
/* ------------------------------------------------------------------ */
/* Rotary inverse frequencies (attention.metal:62-63), 32 fp32 values on the
 * host; the attention op reads them from a device copy. */
int es_rope_inv_freq(float* host_out32);

/* Scratch bytes es_attn_decode needs for a cache of `capacity` rows. Layout
 * (fp32): chain outputs [8,64,256], chain (max, sum) [8,64,2]; the size does
 * not depend on the capacity. */
size_t es_attn_scratch_bytes(int capacity);

/* attn_prepare_qkv_decode (attention.metal:262-313) + decode attention with
 * the output gate, following the reference's routes (model.rs:318-347):
 * attn_decode + attn_gate (32 position chains, fp32 combine) below 1024
 * attended positions, attn_decode_split1 + attn_decode_split2_gate (64
 * chains, bf16 partials) from 1024 on (attention_decode.metal:51-431,
 * 830-891). q_proj [8,512] (query|gate), k_proj/v_proj [2,256]; writes K/V
 * row `position` of kcache/vcache [2, capacity, 256] and
 * gated [8,256] = bf16(bf16(attn) * sigmoid_bf(gate)). Attends to positions
 * 0..position. `blocks` must be 1..1024 and changes nothing (the launch
 * shape is fixed: one block per KV head, chain and query-head pair).
 * query_out (optional) receives the roped queries [8,256]. */
int es_attn_decode(const uint16_t* q_proj, const uint16_t* k_proj, const uint16_t* v_proj,
                   const uint16_t* q_gain, const uint16_t* k_gain, uint16_t* kcache,
                   uint16_t* vcache, int capacity, int position, const float* inv_freq,
                   int blocks, void* scratch, size_t scratch_bytes, uint16_t* gated,
                   uint16_t* query_out, void* stream);

/* ------------------------------------------------------------------ */
/* Vocab head (head_lse.metal:11-98 with rms_norm_bf16, model.rs:290-300) */
/* ------------------------------------------------------------------ */
/* Scratch for es_head_greedy: per-block (max, sum exp) partials. */
size_t es_head_scratch_bytes(int vocab);

/* u = RMSNorm(h)*gain; logits[vocab] = bf16(E u) over the tied table;
 * lse = bf16(log(sum exp) + max) over the bf16 logits; *token = lowest index
 * of max bf16(logit - lse) (docs/protocol.md:44). token/lse are device
 * pointers; norm_out and lse are optional. vocab must be below 2^22. */
int es_head_greedy(const es_q4* embed, const uint16_t* h, const uint16_t* gain,
                   uint16_t* norm_out, uint16_t* logits, void* scratch, size_t scratch_bytes,
                   uint32_t* token, float* lse, void* stream);

/* es_head_greedy for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. The same results as es_head_greedy, with the
 * per-block partials in a device array inside the library (32 KiB per GPU,
 * held until the process ends) instead of caller scratch; allocates nothing.
 * vocab <= ES_HEAD_NOALLOC_MAX_VOCAB, else ES_ERR_INVALID. Every call on one
 * GPU shares that GPU's array: calls that overlap on one GPU (concurrent
 * streams or threads) race. The stream must belong to the current device. */
#define ES_HEAD_NOALLOC_MAX_VOCAB 1048576
int es_head_greedy_noalloc(const es_q4* embed, const uint16_t* h, const uint16_t* gain, uint16_t* norm_out,
                           uint16_t* logits, uint32_t* token, float* lse, void* stream);

/* ------------------------------------------------------------------ */
/* Model weights (weights.rs:11-44 checks; model.rs:41-78 names)        */
/* ------------------------------------------------------------------ */
/* The host weight blob holds every tensor at a 256-byte aligned offset, named
 * as the checkpoint's language_model.model.* tensors. dtype: 0 u32, 1 bf16,
 * 2 f32. Layer l is full attention when l % 4 == 3 (model.rs:51). */
size_t es_weights_total_bytes(int n_layers, int vocab);
int es_weights_tensor_count(int n_layers);
int es_weights_tensor_info(int n_layers, int vocab, int index, char* name, int name_len,
                           uint64_t* offset, uint64_t* bytes, int* dtype);
/* Checkpoint shape of tensor `index` (model.rs:41-78; conv1d is [6144,4,1]):
 * writes up to max_dims sizes and returns the number of dims, or a negative
 * ES_ERR_* code. */
int es_weights_tensor_shape(int n_layers, int vocab, int index, int64_t* dims, int max_dims);
/* Seeded random-init model (Q4 of N(0,0.02) weights, see es_weights.hpp). */
int es_weights_random(int n_layers, int vocab, uint64_t seed, void* blob, size_t bytes,
                      int threads);

/* Checkpoint directory (Weights::load, weights.rs:11-15): config.json's
 * text_config must have hidden_size 1024, num_hidden_layers 24 and
 * vocab_size 248320, else ES_ERR_INVALID "unsupported model configuration".
 * Writes the model shape (24, 248320). */
int es_checkpoint_config(const char* model_dir, int* n_layers, int* vocab);
/* Fills a weight blob (es_weights_total_bytes(n_layers, vocab) bytes, host
 * memory) from every *.safetensors file of model_dir, checked as
 * Weights::load / take / linear / done do (weights.rs:16-53, model.rs:38-79):
 * only language_model.model.* tensors, dtypes U32/F32/BF16, byte ranges
 * inside the file and equal to the shape's size, no duplicates, exactly the
 * model's text tensor count (694 for 24 layers), each tensor present with the
 * model's shape and dtype. Errors carry the reference's messages
 * ("missing <name>", "wrong shape/dtype for <name>", ...). */
int es_checkpoint_load(const char* model_dir, int n_layers, int vocab, void* blob, size_t bytes);

/* ------------------------------------------------------------------ */
/* Engine (Model::load / generate / cancelled, model.rs:28-180)        */
/* ------------------------------------------------------------------ */
typedef struct es_engine es_engine;

/* Model::load (model.rs:37-92) from a host blob; capacity = KV positions
 * (reference CAPACITY 262144, model.rs:8). NULL on failure. */
es_engine* es_engine_create(const void* blob, size_t bytes, int n_layers, int vocab,
                            int capacity);
void es_engine_destroy(es_engine* e);

/* Model::generate (model.rs:97-122): reset=1 consumes prompt[len] (len>0)
 * and emits max_tokens greedy ids; reset=0 requires len==0 and first consumes
 * the last emitted token. out[max_tokens] is host memory. On error the request
 * is rejected with the reference's messages; after a device error or a
 * cancellation the state is reset (model.rs:175-178). */
int es_engine_generate(es_engine* e, const uint32_t* prompt, int len, int max_tokens, int reset,
                       uint32_t* out);

/* Prompt consumption of es_engine_generate (model.rs:106-109, CHUNK 2048
 * model.rs:7). With chunk_rows >= 2 (default 4096, at most 65536) the
 * n = len-1 prompt tokens are consumed as the reference's forwards of 2048
 * rows from position 0 would be: the rows of full forwards take the batched
 * GEMM and flash attention, run here in chunks of at most chunk_rows rows
 * (their results do not depend on the grouping); the last, shorter forward of
 * r = n mod 2048 rows, when r < 33, is routed as Model::linear routes it
 * (model.rs:189-198): r == 1 runs the decode kernels (forward with rows == 1),
 * otherwise each linear with r below es_linear_row_limit runs as
 * es_q4_matvec_rows. chunk_rows 0 instead replays one decode step per prompt
 * token (not the reference's arithmetic). Consecutive chunks run on two
 * streams, one layer apart. Batched prefill allocates two sets of chunk
 * buffers (about 67 KB per row each) on first use. */
int es_engine_set_prefill(es_engine* e, int chunk_rows);

/* 1 when the engine's decode steps use the XCD-cooperative kernels (the
 * layer's MLP in one launch whose blocks exchange activations within each
 * XCD; chosen at es_engine_create after a placement probe), 0 when they use
 * one launch per dependency; -ES_ERR_INVALID for a null engine. Both give the
 * same bits. No reference counterpart. */
int es_engine_xcd_kernels(const es_engine* e);
/* Selects the decode kernels: on=1 the XCD-cooperative ones (ES_ERR_INVALID
 * when the placement probe ruled them out), on=0 one launch per dependency.
 * Call between requests; the engine's cached decode graphs are rebuilt. No
 * reference counterpart: lets tests hold the two kernel sets to the same
 * bits. */
int es_engine_set_xcd_kernels(es_engine* e, int on);
/* Test hook for the failure path of the XCD-cooperative kernels' exchange
 * waits, forced from the host so every kernel still exits normally. mode 1
 * sets the device error word: every wait of the following launches gives up
 * at once. mode 2 moves one block's exchange count away from its XCD's, so
 * the waits on that block's words run to their spin limit (tens of
 * milliseconds) and then every other wait gives up. The next request fails
 * with ES_ERR_DEVICE ("decode kernels: an XCD exchange wait timed out"),
 * after which the engine has cleared the error word, the counts and the
 * exchange words, and the request after it runs normally. ES_ERR_INVALID
 * when the XCD-cooperative kernels are off. No reference counterpart. */
int es_engine_inject_exchange_fault(es_engine* e, int mode);

/* How the last reset request consumed its prompt: batched chunks of
 * full-forward rows, rows of the routed last forward (0 or 2 .. 32), and
 * rows run on the decode kernels (0 or 1; every row with chunk_rows 0). No
 * reference counterpart: lets tests and callers see the routing. */
int es_engine_prompt_split(const es_engine* e, int* chunks, int* routed_rows, int* decode_rows);

/* cancelled.store(true) (main.rs:24): the running request stops at its next
 * step boundary, drains, resets and fails with ES_ERR_CANCELLED. */
void es_engine_cancel(es_engine* e);
void es_engine_clear_cancel(es_engine* e);
int es_engine_position(const es_engine* e);

/* Teacher forcing (docs/protocol.md:61-63): step i consumes tokens[i]; the
 * greedy pick after it goes to argmax[i]; logits (optional host [n, vocab]). */
int es_engine_forced_decode(es_engine* e, const uint32_t* tokens, int n, uint32_t* argmax,
                            uint16_t* logits);

/* State handoff to/from host memory. which: 0 K cache, 1 V cache; KV data is
 * [2 heads, count, 256] bf16 for positions pos0..pos0+count-1. */
int es_engine_read_kv(es_engine* e, int layer, int which, int pos0, int count, void* host);
int es_engine_write_kv(es_engine* e, int layer, int which, int pos0, int count,
                       const void* host);
/* GDN layer ring [4,6144] bf16 and state [16,128,128] fp32; NULL skips one. */
int es_engine_read_gdn(es_engine* e, int layer, void* ring, void* state);
int es_engine_write_gdn(es_engine* e, int layer, const void* ring, const void* state);
/* Declare that `position` tokens are consumed and `pending` is next. */
int es_engine_set_position(es_engine* e, int position, uint32_t pending);
/* Synthetic context of `length` consumed tokens (benchmarks). */
int es_engine_fill_synthetic(es_engine* e, int length, uint64_t seed, uint32_t pending);

/* Timing with HIP events on the engine stream. */
int es_engine_time_decode(es_engine* e, int steps, int warmup, double* ms_total);
/* which: 0 = both attention launches, 1 = scores with the chains, 2 = merge.
 * layer < 0 rotates over every attention layer (cold KV caches, as in a
 * decode step); layer >= 0 repeats that layer. */
int es_engine_time_attention(es_engine* e, int layer, int reps, int which, double* ms_avg);
int es_engine_time_head(es_engine* e, int reps, double* ms_avg);
/* The `blocks` value the engine passes to the attention launch (constant). */
int es_engine_splits_for(int length);

#ifdef __cplusplus
}
#endif
#endif
