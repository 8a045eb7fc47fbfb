// Host-side launchers for the decode kernels. Every launcher checks the
// shapes its kernel assumes and returns hipErrorInvalidValue (without
// launching) when they do not hold; device pointers are caller-owned.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "es_device.hpp"

namespace es {

// ---- linear (Q4 affine group 64), k_linear.hip ----
// RMSNorm(x)*gain (K=1024) followed by up to four projections sharing the
// normalised input. When embed.w is set, x is instead the bf16 embedding row
// of the token in st->token (or token_val when st is null); block 0 writes
// that row to h_out. With ring0 set, output 0 is a 4-slot ring [4, n0] and the
// slot (pos & 3) is written.
struct NormMultiArgs {
  Q4 m[4];
  uint16_t* y[4];
  int count;
  int ring0;
  const uint16_t* x;
  const float* dpart;       // optional [8, 1024]: x := bf16(x + bf16(pairwise sum of dpart)), written to h_out
  const uint16_t* gain;
  uint16_t* norm_out;
  Q4 embed;
  uint16_t* h_out;
  uint32_t token_val;
  const StepState* st;
  int pos_val;
};
hipError_t launch_norm_multi(const NormMultiArgs& a, hipStream_t s);

// RMSNorm(x)*gain then act = SwiGLU(gate u, up u) (K=1024).
hipError_t launch_norm_gate_up(const Q4& gate, const Q4& up, const uint16_t* x,
                               const uint16_t* gain, uint16_t* norm_out, uint16_t* act,
                               hipStream_t s);

// Engine path: h_new = bf16(h_old + bf16(pairwise sum of nparts head
// partials [nparts, 1024])) (8: o_proj, 16: GDN out_proj), then as above
// on h_new. h_new must not alias h_old.
hipError_t launch_norm_gate_up_parts(const Q4& gate, const Q4& up, const uint16_t* h_old,
                                     const float* part, int nparts, uint16_t* h_new,
                                     const uint16_t* gain, uint16_t* act, hipStream_t s);

// y = bf16(W x) or, with residual, y = bf16(residual + bf16(W x)). x bf16[K].
// K == 1024 or 1024 < K <= 4096 with K % 64 == 0. y may alias residual.
hipError_t launch_qmv(const Q4& w, const uint16_t* x, const uint16_t* residual, uint16_t* y,
                      float* y_f32, hipStream_t s);
// The same for `rows` token rows (qmv_q4 with M rows): x [rows, K], residual
// and y [rows, N]; each row has the M = 1 arithmetic. y_f32 only for rows == 1.
hipError_t launch_qmv_rows(const Q4& w, const uint16_t* x, int rows, const uint16_t* residual,
                           uint16_t* y, float* y_f32, hipStream_t s);
// Row count from which a batched linear of an [n, k] matrix takes the GEMM
// (qmm_q4_nax) instead of qmv_q4 rows: 33, 25 or 13 by shape (model.rs:189-192,
// MLX 0.32.4 get_qmv_batch_limit for the reference's GPU family).
int qmv_row_limit(int n, int k);

// add_bf16 (linear.metal:372-379): out = bf16(a + b) over count elements;
// out may alias a or b.
hipError_t launch_add_bf16(const uint16_t* a, const uint16_t* b, int count, uint16_t* out, hipStream_t s);

// Embedding row: out = bf16(scale*q + bias) for token *token_dev.
hipError_t launch_embedding(const Q4& table, const uint32_t* token_dev, uint16_t* out,
                            hipStream_t s);

// ---- Gated DeltaNet, k_gdn.hip ----
struct GdnRecurArgs {
  const uint16_t* ring;     // [4, 6144] raw projected qkv, slot = position & 3
  const uint16_t* conv_w;   // [6144, 4]
  const uint16_t* ab;       // a[16] then b[16] raw projections
  const float* a_log;       // [16]
  const uint16_t* dt_bias;  // [16]
  float* state;             // [16, 128 v, 128 k] in place
  uint16_t* y;              // [2048]
  uint16_t* qkv_out;        // optional [6144]: normalised q|k and activated v
  float* g_out;             // optional [16]
  uint16_t* beta_out;       // optional [16]
  const StepState* st;
  int pos_val;
};
hipError_t launch_gdn_recur(const GdnRecurArgs& a, hipStream_t s);

// Engine path: recurrence + gated RMSNorm + out_proj partials per head
// (part[h][r] = the head's 128 columns of row r, the four slice partials
// combined pairwise); the next launch adds the 16 partials pairwise.
struct GdnOutArgs {
  GdnRecurArgs r;           // y, qkv_out, g_out, beta_out unused
  const uint16_t* z;        // [2048] output-gate projection
  const uint16_t* norm_w;   // [128]
  Q4 out;                   // out_proj [1024, 2048]
  float* part;              // [16, 1024]
};
hipError_t launch_gdn_recur_out(const GdnOutArgs& a, hipStream_t s);

// Gated RMSNorm of y by z (per 128-wide head) feeding out_proj (K=2048) with
// the residual add: h = bf16(h + bf16(W gated)). gated_out (optional) receives
// the gated vector from block 0.
hipError_t launch_gdn_gate_out(const Q4& w, const uint16_t* y, const uint16_t* z,
                               const uint16_t* norm_w, uint16_t* h, uint16_t* gated_out,
                               hipStream_t s);

// ---- attention, k_attention.hip ----
// Decode attention follows the reference's two routes (model.rs:327-347):
// below 1024 cached positions 32 interleaved position chains combined in
// fp32 (sdpa_vector), from 1024 on 64 chains whose outputs are rounded to
// bf16 before the gated merge (sdpa_vector_2pass_1 + split2_gate). Two
// launches: scores with the per-chain online softmax, then merge + gate.
constexpr int kAttnRouteSplit = 1024;  // first length served by 64 chains
constexpr int kAttnMaxChains = 64;
struct AttnArgs {
  const uint16_t* q_proj;   // [8, 512] query|gate per head
  const uint16_t* k_proj;   // [2, 256]
  const uint16_t* v_proj;   // [2, 256]
  const uint16_t* q_gain;   // [256]
  const uint16_t* k_gain;   // [256]
  uint16_t* kcache;         // [2, capacity, 256]
  uint16_t* vcache;         // [2, capacity, 256]
  int capacity;
  const float* inv_freq;    // [32] rotary inverse frequencies
  float* part_o;            // [8, 64, 256] unnormalised chain outputs
  float* part_ml;           // [8, 64, 2] chain (max, sum)
  int blocks;               // accepted for the C ABI (1..1024); no launch depends on it
  uint16_t* gated;          // [8, 256]
  uint16_t* query_out;      // optional [8, 256] roped queries
  const StepState* st;
  int pos_val;
};
size_t attn_scratch_bytes(int capacity);
void attn_bind_scratch(AttnArgs& a, void* scratch);
hipError_t launch_attn_fused(const AttnArgs& a, hipStream_t s);
hipError_t launch_attn_merge(const AttnArgs& a, hipStream_t s);
// Engine path: merge + gate, then o_proj partials per head (part[h][r] = the
// head's 256 columns of row r, its eight slice partials combined pairwise);
// the next launch adds the 8 partials pairwise. o_sb: o_proj's group words by
// head ([8, 1024, 4], launch_pack_out_pairs: head h spans groups 4h .. 4h+3).
hipError_t launch_attn_merge_out(const AttnArgs& a, const Q4& o, const uint32_t* o_sb, float* part,
                                 hipStream_t s);

// ---- XCD-cooperative decode kernels, k_fused.hip ----
// The MLP of a layer in one 256-block launch (blocks of one XCD exchange
// activations through its L2): h_mid = bf16(h_old + bf16(pairwise sum of the
// 8 mixer partials)) (k_gdn_xcd's head pairs, or k_attn_merge_out's o_proj
// heads; nparts must be 8), post
// RMSNorm, gate/up, SwiGLU, then dpart[x][r] = octet x's share of the down
// row r's sum (x = 0..7). The consumer adds them: h = bf16(h_mid +
// bf16(pairwise sum over x of dpart[x][r])), the down projection's residual
// epilogue bit for bit.
struct MlpXcdArgs {
  Q4 gate, up, down;
  const uint2* gu_sb;       // [3584, 16] (gate, up) scale|bias<<16 words (launch_pack_sb2)
  const uint32_t* down_sb;  // [8 octets, 1024, 8] scale|bias<<16 words (launch_pack_down_octets)
  const uint16_t* h_old;    // [1024] residual stream before the mixer
  const float* part;        // [nparts, 1024] mixer partials
  uint16_t* h_mid;          // [1024] written: stream after the mixer
  const uint16_t* gain;     // post-attention norm [1024]
  float* dpart;             // [8, 1024] down partials
  uint32_t* xact;           // [8, 512] activation exchange words: bf16 | tag << 16 (zeroed at start-up)
  uint32_t* flags;          // [8, 32] per-block exchange counts (zero at start-up)
  uint32_t* err;            // error word: 2 = an exchange wait hit its limit
};
hipError_t launch_mlp_xcd(const MlpXcdArgs& a, int nparts, hipStream_t s);
// A Gated DeltaNet layer up to its out_proj head partials in one 256-block
// launch (k_norm_multi + k_gdn_recur_out, bit for bit): the input is the
// embedding row of st->token (embed.w set) or x + the down partials dpart of
// the previous layer's k_mlp_xcd; h_out (block 0) receives it.
struct GdnXcdArgs {
  const uint16_t* x;        // [1024] stream after the previous layer's mixer
  const float* dpart;       // [8, 1024] the previous layer's down partials
  Q4 embed;                 // layer 0: the token's embedding row is the input
  uint16_t* h_out;          // [1024] the layer input
  const uint16_t* gain;     // input norm [1024]
  Q4 qkv, z, a, b, out;
  // scale|bias<<16 words of the same matrices (launch_pack_sb): qkv [6144,16],
  // z [2048,16], a then b [2,16,16]; out per XCD [8, 1024, 4] (the groups of
  // the XCD's head pair, launch_pack_out_pairs)
  const uint32_t* qkv_sb;
  const uint32_t* z_sb;
  const uint32_t* ab_sb;
  const uint32_t* out_sb;
  const uint16_t* conv_w;   // [6144, 4]
  const uint16_t* norm_w;   // [128]
  const uint16_t* dt_bias;  // [16]
  const float* a_log;       // [16]
  uint16_t* ring;           // [4, 6144]
  float* state;             // [16, 128, 128]
  float* part;              // [8, 1024] out_proj partials of the head pairs (2x, 2x+1)
  uint32_t* xbuf;           // [8 XCDs][2 heads][648] exchange words: bf16 | tag << 16 (zeroed at start-up)
  uint32_t* flags;          // [8, 32] per-block exchange counts (shared with k_mlp_xcd)
  uint32_t* err;            // error word
  const StepState* st;
};
hipError_t launch_gdn_xcd(const GdnXcdArgs& a, hipStream_t s);
// Packed group words for the XCD kernels: out[i] = s[i] | b[i] << 16 (the
// bf16 scale and bias of one Q4 group), n groups; pack_sb2 interleaves two
// matrices of the same shape: out[i] = (s0|b0<<16, s1|b1<<16).
hipError_t launch_pack_sb(const uint16_t* s, const uint16_t* b, uint32_t* out, size_t n, hipStream_t st);
hipError_t launch_pack_sb2(const uint16_t* s0, const uint16_t* b0, const uint16_t* s1, const uint16_t* b1,
                           uint2* out, size_t n, hipStream_t st);
// The down projection's words by XCD octet: out[x][r][w] = the word of group
// 4x + w (w < 4) and, for x < 6, of group 32 + 4x + w - 4 (w >= 4) of row r
// (K = 3584: 56 groups per row), so each XCD reads one contiguous block.
hipError_t launch_pack_down_octets(const uint16_t* s, const uint16_t* b, uint32_t* out, hipStream_t st);
// out_proj's words by head pair: out[x][r][w] = the word of group 4x + w of
// row r (K = 2048: 32 groups per row; heads 2x, 2x+1 span groups 4x .. 4x+3).
hipError_t launch_pack_out_pairs(const uint16_t* s, const uint16_t* b, uint32_t* out, hipStream_t st);
// out[b] = XCC_ID of block b of a 256-block launch.
hipError_t launch_xcc_probe(uint32_t* out, hipStream_t s);

// ---- batched prefill, k_prefill.hip ----
// Y[m,N] = bf16(X[m,K] . W^T) with W dequantised to bf16 per weight, fp32
// accumulation (qmm_q4_nax); with residual: Y = bf16(R + bf16(X . W^T)).
// K a multiple of 64. Y may alias R.
hipError_t launch_q4_gemm(const Q4& w, const uint16_t* x, int m, const uint16_t* residual, uint16_t* y,
                          hipStream_t s);
// MLP gate/up linears with SwiGLU in one GEMM (the same results as the two
// row-batched linears followed by swiglu_bf16): act [m, gate.n].
hipError_t launch_q4_gemm_swiglu(const Q4& gate, const Q4& up, const uint16_t* x, int m, uint16_t* act,
                                 hipStream_t s);
// Linears sharing one input, stacked along N (q|k|v, qkv|z|a|b): segment s
// is Y_s[m, w[s].n] = bf16(X . W_s^T), bit for bit the separate linears.
struct WideGemmArgs {
  Q4 w[4];
  uint16_t* y[4];
  int nstart[5];  // first column of each segment; nstart[nseg] = total N
  int nseg;
  const uint16_t* x;
  int m;
};
hipError_t launch_q4_gemm_stacked(const Q4* w, uint16_t* const* y, int nseg, const uint16_t* x, int m,
                                  hipStream_t s);
// Row forms of the decode operators (m rows = consecutive positions
// pos0 .. pos0+m-1), each with the decode kernels' arithmetic per row.
hipError_t launch_embed_rows(const Q4& e, const uint32_t* tokens, int m, uint16_t* h, hipStream_t s);
hipError_t launch_rmsnorm_rows(const uint16_t* x, const uint16_t* gain, int m, uint16_t* out, hipStream_t s);
hipError_t launch_swiglu_rows(const uint16_t* gate, const uint16_t* up, int count, uint16_t* act,
                              hipStream_t s);
struct GdnPrepRowsArgs {
  const uint16_t* raw;      // [m, 6144] projected q|k|v before the convolution
  uint16_t* ring;           // [4, 6144] raw rows of the last positions, slot = position & 3
  const uint16_t* conv_w;   // [6144, 4]
  const uint16_t* a_proj;   // [m, 16]
  const uint16_t* b_proj;   // [m, 16]
  const float* a_log;       // [16]
  const uint16_t* dt_bias;  // [16]
  int pos0, m;
  uint16_t *q, *k, *v;      // [m, 16, 128] normalised q, k and activated v
  float *g, *beta;          // [m, 16]
};
// Convolution, activation, q/k normalisation and gates of every row, then
// the ring takes the chunk's last raw rows.
hipError_t launch_gdn_prep_rows(const GdnPrepRowsArgs& a, hipStream_t s);
// Delta-rule recurrence over the m rows in order; y [m, 2048] bf16.
hipError_t launch_gdn_recur_rows(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                                 const float* beta, int m, float* state, uint16_t* y, hipStream_t s);
// The reference's GDN interface over a history [3, 6144] (GDN_INTERFACE.md:
// 12-18): gdn_conv (conv [rows,6144]), gdn_history (history takes the last
// three raw rows), gdn_prepare (q, k normalised in place in conv; g fp32 and
// beta bf16 [rows,16]) and gdn_recur over the normalised conv buffer.
hipError_t launch_gdn_conv_hist(const uint16_t* raw, const uint16_t* history, const uint16_t* conv_w,
                                int rows, uint16_t* conv, hipStream_t s);
hipError_t launch_gdn_history(const uint16_t* raw, int rows, uint16_t* history, hipStream_t s);
hipError_t launch_gdn_prepare_hist(uint16_t* conv, const uint16_t* a_proj, const uint16_t* b_proj,
                                   const float* a_log, const uint16_t* dt_bias, int rows, float* g,
                                   uint16_t* beta, hipStream_t s);
hipError_t launch_gdn_recur_conv(const uint16_t* conv, const float* g, const uint16_t* beta, int rows,
                                 float* state, uint16_t* y, hipStream_t s);
hipError_t launch_gdn_norm_gate_rows(const uint16_t* y, const uint16_t* z, const uint16_t* norm_w, int m,
                                     uint16_t* out, hipStream_t s);
struct AttnPrepRowsArgs {
  const uint16_t* qg;       // [m, 4096] q|gate per head
  const uint16_t* k;        // [m, 512]
  const uint16_t* v;        // [m, 512]
  const uint16_t* q_gain;   // [256]
  const uint16_t* k_gain;   // [256]
  const float* inv_freq;    // [32]
  int pos0, m;
  uint16_t* qr;             // [m, 8, 256] normalised, roped queries
  uint16_t* kcache;         // [2, capacity, 256]
  uint16_t* vcache;
  int capacity;
};
hipError_t launch_attn_prep_rows(const AttnPrepRowsArgs& a, hipStream_t s);
// Causal GQA attention of the m queries at positions pos0.. over cache rows
// 0 .. pos0+m-1: o [m, 8, 256] bf16 (attn_prefill).
hipError_t launch_attn_prefill(const uint16_t* qr, const uint16_t* kcache, const uint16_t* vcache, int pos0,
                               int m, int capacity, uint16_t* o, hipStream_t s);
hipError_t launch_attn_gate_rows(const uint16_t* o, const uint16_t* qg, int m, uint16_t* gated,
                                 hipStream_t s);

// ---- vocab head, k_head.hip ----
struct HeadArgs {
  Q4 embed;                 // tied table [vocab, 1024]
  const uint16_t* h;        // [1024]
  const float* dpart;       // optional [8, 1024]: h := bf16(h + bf16(pairwise sum of dpart))
  const uint16_t* gain;     // final norm [1024]
  uint16_t* norm_out;       // optional
  uint16_t* logits;         // [vocab] bf16
  float* part;              // [blocks, 2] (max, sumexp)
  uint32_t* token_out;      // written by the tail (may be null)
  float* lse_out;           // optional
  StepState* st;            // optional: advances pos/step, stores token, out_tokens[step]
  uint32_t* out_tokens;     // optional with st
};
int head_blocks(int vocab);
size_t head_scratch_bytes(int vocab);
hipError_t launch_head(const HeadArgs& a, hipStream_t s);
// launch_head with the block partials in a file-scope device array instead
// of a.part (ignored): allocates nothing; vocab <= head_noalloc_max_vocab().
int head_noalloc_max_vocab();
hipError_t launch_head_noalloc(HeadArgs a, hipStream_t s);
// greedy_bf16 over bf16 logits in memory: the head's LSE and tie rule
// (part: head_scratch_bytes(count)); token and lse (optional) on the device.
hipError_t launch_greedy(const uint16_t* logits, int count, float* part, uint32_t* token, float* lse,
                         hipStream_t s);

// Prompt step epilogue: pos += 1, token = prompt[pos].
hipError_t launch_advance(StepState* st, const uint32_t* prompt, hipStream_t s);
// st->token = *src (teacher forcing from a device token list).
hipError_t launch_set_token(StepState* st, const uint32_t* src, hipStream_t s);
// Fill with N(0, sigma) bf16 / fp32 values from a counter-based generator.
hipError_t launch_fill_normal_bf16(uint16_t* dst, size_t n, float sigma, uint64_t seed,
                                   hipStream_t s);
// Device-to-device copy of `bytes` (a multiple of 16) by a plain kernel.
hipError_t launch_copy16(void* dst, const void* src, size_t bytes, hipStream_t s);
// Streaming read of `bytes` (a multiple of read_granule()) by global->LDS DMA;
// out: read_out_bytes() of device scratch.
size_t read_out_bytes();
size_t read_granule();
hipError_t launch_read(const void* src, size_t bytes, void* out, hipStream_t s);
hipError_t launch_fill_normal_f32(float* dst, size_t n, float sigma, uint64_t seed,
                                  hipStream_t s);

}  // namespace es
