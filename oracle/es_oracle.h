/*
 * es_oracle.h -- CPU restatement of the reference decode-step arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * decode engine. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker or as the timed CPU
 * baseline. The engine never links, loads or calls it.
 *
 * Every function restates one reference kernel; the citation names the Metal
 * source (paths relative to the reference checkout). bf16 values are passed
 * as raw uint16_t bit patterns; "bf16(x)" means round-to-nearest-even of an
 * fp32 value, taken at exactly the reference's rounding points. The
 * reference's fp32 accumulation order is not fully specified (Metal simd_sum
 * trees and FMA contraction are left to its compiler), so every reduction here
 * follows one stated fp32 order -- the one the HIP kernels use -- which makes
 * the parity tests bitwise where the algorithms coincide. exp/log/sin/cos are
 * the series evaluations in es_oracle.c (the kernels evaluate the same
 * steps). Compiled with -ffp-contract=off: FMAs appear only where fmaf is
 * written. Decode attention keeps the reference's own algorithm (32 or 64
 * interleaved position chains, bf16 chain outputs at and above 1024
 * positions) with one stated order for each score, chain update and merge.
 *
 * Pinning (tests/test_oracle_*.py, tests/test_golden.py):
 *   bf16 RNE, widening ............. exhaustive / 2M patterns vs torch, ties
 *   exp, log / sin, cos ............ <= 2 ulp / <= 2.5e-7 vs fp64 libm, specials
 *   sigmoid/softplus (bf16 steps) .. all 65,536 bf16 inputs vs fp64 model
 *   rotary frequencies ............. closed form 1e7^(-i/32)
 *   Q4 matvec / embedding .......... integer-dot exactness, zero-code closed
 *                                    form, fp64 dequant brute force, linearity
 *   RMSNorm ........................ constant-vector closed form (bitwise), fp64
 *   GDN conv/prepare/recur/gate .... delta-rule invariants, fp64 recurrence
 *   attention prepare (RoPE) ....... position-0 identity, fp64 rotation, norms
 *   attention decode/split/merge ... N=1, equal keys, dominant key, fp64 route
 *                                    model, split vs single, chain states
 *   greedy ......................... planted maxima, exact ties, fp64 lse
 * No function is "parity unpinned".
 */
#ifndef ES_ORACLE_H
#define ES_ORACLE_H
#include <stdint.h>
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- model constants (reference model.rs:7-9, 41-78) ---- */
#define EO_HIDDEN 1024
#define EO_FFN 3584
#define EO_GDN_HEADS 16
#define EO_GDN_DK 128
#define EO_GDN_CONV 6144
#define EO_ATT_QHEADS 8
#define EO_ATT_KVHEADS 2
#define EO_ATT_DIM 256
#define EO_SPLIT_BLOCKS 64

/* ---- numerics ---- */
float eo_bf16_to_f32(uint16_t b);
uint16_t eo_f32_to_bf16(float f);
float eo_round_bf16(float f);
void eo_f32_to_bf16_array(const float* in, uint16_t* out, size_t n);
void eo_bf16_to_f32_array(const uint16_t* in, float* out, size_t n);
float eo_exp(float x);          /* series exp (degree-7 Taylor after ln2 reduction) */
float eo_log(float x);          /* series log (atanh series), positive normal x */
void eo_sincos(float x, float* s, float* c); /* double quadrant reduction + Taylor */
float eo_sigmoid_bf(float x);   /* linear.metal:389-395, gdn.metal:10-15 */
float eo_softplus_bf(float x);  /* gdn.metal:19-29 */
float eo_rope_inv_freq(int pair); /* attention.metal:62-63 */

/* ---- linear (Q4 affine, group 64) ---- */
/* embedding_q4, linear.metal:11-24 */
void eo_embedding(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases,
                  int K, uint32_t token, uint16_t* out);
/* qmv_q4 walk, linear.metal:28-73; y_f32 (optional) receives the pre-round sum */
void eo_q4_matvec(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases,
                  int N, int K, const uint16_t* x, uint16_t* y, float* y_f32);
/* qmv_add_q4, linear.metal:77-123: y = bf16(residual + bf16(qmv)); y may alias residual */
void eo_q4_matvec_add(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases,
                      int N, int K, const uint16_t* x, const uint16_t* residual, uint16_t* y);
/* rms_norm_bf16, linear.metal:300-331 (and the RMS prologue of
 * linear_input_norm.metal:38-63 / linear_norm.metal:26-50) */
void eo_rms_norm(const uint16_t* x, const uint16_t* gain, int cols, float eps, uint16_t* out);
/* swiglu_bf16, linear.metal:382-396 */
void eo_swiglu(const uint16_t* gate, const uint16_t* up, int n, uint16_t* out);

/* ---- Gated DeltaNet ---- */
/* gdn_conv_prepare_decode, gdn.metal:121-171 (== gdn_input.metal:157-205).
 * raw[6144] projected qkv; history[3*6144] updated in place; conv_out[6144];
 * a,b[16] projected gates; g[16] fp32; beta[16] bf16. */
void eo_gdn_conv_prepare(const uint16_t* raw, uint16_t* history, const uint16_t* conv_w,
                         const uint16_t* a, const uint16_t* b, const float* a_log,
                         const uint16_t* dt_bias, uint16_t* conv_out, float* g, uint16_t* beta);
/* gdn_recur, gdn.metal:176-228, T=1: state[16,128v,128k] in place, y[2048] */
void eo_gdn_recur(const uint16_t* conv, const float* g, const uint16_t* beta,
                  float* state, uint16_t* y);
/* gdn_norm_gate, gdn.metal:230-255 */
void eo_gdn_norm_gate(const uint16_t* y, const uint16_t* z, const uint16_t* w, uint16_t* out);
/* The same three steps over T consecutive tokens (gdn_conv + gdn_history +
 * gdn_prepare, gdn_recur, gdn_norm_gate with rows = T): token t's results are
 * those of the single-token functions called in token order. raw, conv_out
 * [T,6144]; a, b, beta [T,16] bf16; g [T,16]; y, z, out [T,2048]. */
void eo_gdn_conv_prepare_rows(const uint16_t* raw, uint16_t* history, const uint16_t* conv_w,
                              const uint16_t* a, const uint16_t* b, const float* a_log,
                              const uint16_t* dt_bias, int T, uint16_t* conv_out, float* g,
                              uint16_t* beta);
void eo_gdn_recur_rows(const uint16_t* conv, const float* g, const uint16_t* beta, int T,
                       float* state, uint16_t* y);
void eo_gdn_norm_gate_rows(const uint16_t* y, const uint16_t* z, const uint16_t* w, int T,
                           uint16_t* out);

/* ---- attention ---- */
/* attn_prepare_qkv_decode, attention.metal:262-313. q_proj[8*512], k[512], v[512];
 * writes query[8*256] and cache row `position` of kcache/vcache [2,capacity,256]. */
void eo_attn_prepare(const uint16_t* q_proj, const uint16_t* k, const uint16_t* v,
                     const uint16_t* q_gain, const uint16_t* k_gain, uint16_t* query,
                     uint16_t* kcache, uint16_t* vcache, int position, int capacity);
/* attn_decode = sdpa_vector<bf16,256>, attention_decode.metal:51-213: out[8*256] */
void eo_attn_decode_single(const uint16_t* query, const uint16_t* kcache, const uint16_t* vcache,
                           int length, int capacity, uint16_t* out);
/* attn_decode_split1 = sdpa_vector_2pass_1, attention_decode.metal:215-431, 64 blocks:
 * partials bf16 [8,64,256], sums/maxs fp32 [8,64] */
void eo_attn_decode_split(const uint16_t* query, const uint16_t* kcache, const uint16_t* vcache,
                          int length, int capacity, uint16_t* partials, float* sums, float* maxs);
/* attn_decode_split2_gate, attention_decode.metal:830-891 */
void eo_attn_split_merge_gate(const uint16_t* partials, const float* sums, const float* maxs,
                              const uint16_t* q_proj, uint16_t* gated);
/* attn_gate, attention.metal:133-151 */
void eo_attn_gate(const uint16_t* attn, const uint16_t* q_proj, uint16_t* gated);
/* model.rs:327-347 route: single pass below 1024, split at and above. gated[8*256] */
void eo_attn_decode_gated(const uint16_t* query, const uint16_t* kcache, const uint16_t* vcache,
                          int length, int capacity, const uint16_t* q_proj, uint16_t* gated);

/* ---- head ---- */
/* head_lse_g8 + head_lse_tail, head_lse.metal:11-98, over bf16 logits[n] */
uint32_t eo_greedy(const uint16_t* logits, int n, float* lse_out);

/* ---- full decode step (model.rs:228-307 rows==1, :308-350) ---- */
typedef struct {
  const uint32_t* w; const uint16_t* s; const uint16_t* b; int n, k;
} eo_linear;

typedef struct {
  int is_attention;
  const uint16_t* input_norm; const uint16_t* post_norm;
  eo_linear gate, up, down;
  /* GDN */
  eo_linear qkv, z, a, b, out;
  const uint16_t* conv_w; const uint16_t* gdn_norm; const uint16_t* dt_bias; const float* a_log;
  /* attention */
  eo_linear q, k, v, o;
  const uint16_t* q_norm; const uint16_t* k_norm;
} eo_layer;

typedef struct {
  int n_layers; int vocab;
  eo_linear embed; const uint16_t* final_norm;
  eo_layer layers[64];
} eo_model;

typedef struct {
  int capacity;
  uint16_t* history[64];   /* GDN layers: [3,6144] bf16 (reference layout) */
  float* state[64];        /* GDN layers: [16,128,128] fp32 */
  uint16_t* kcache[64];    /* attention layers: [2,capacity,256] */
  uint16_t* vcache[64];
} eo_state;

/* One decode step at absolute position `position` consuming `token`.
 * If logits != NULL the bf16 logits [vocab] are written there (else scratch).
 * Returns the greedy token; want_head=0 skips the LM head (prompt consumption)
 * and returns 0. hidden_out (optional) receives the final pre-norm hidden [1024]. */
uint32_t eo_model_step(const eo_model* m, eo_state* st, uint32_t token, int position,
                       int want_head, uint16_t* logits, uint16_t* hidden_out);

int eo_num_threads(void);
void eo_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
