/*
 * es_oracle.c -- CPU restatement of the reference decode-step arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and timed CPU baseline); the HIP
 * engine never links or calls this file. See es_oracle.h for the contract and
 * the pinning status of each function. Citations are to the reference
 * checkout (source/src/kernels/ Metal files, source/src/model.rs).
 *
 * SIMD-group reductions (simd_sum over 32 lanes) are restated as xor
 * butterflies; their hardware order is not specified by the reference.
 */
#include "es_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* numerics                                                            */
/* ------------------------------------------------------------------ */
float eo_bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t eo_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float eo_round_bf16(float f) { return eo_bf16_to_f32(eo_f32_to_bf16(f)); }

void eo_f32_to_bf16_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = eo_f32_to_bf16(in[i]);
}
void eo_bf16_to_f32_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = eo_bf16_to_f32(in[i]);
}

#define BF(x) eo_round_bf16(x)
#define F(b) eo_bf16_to_f32(b)

/* ---- series math, step for step the same evaluation as the kernels ----
 * exp: x = n ln2 + r, |r| <= ln2/2 (ln2 split in a 12-bit-exact head and a
 * tail), degree-7 Taylor polynomial of e^r by Horner with fma, times 2^n.
 * Inputs <= -86 give 0 so every result is a normal number. */
float eo_exp(float x) {
  if (!(x > -86.0f)) return 0.0f;
  if (x > 88.72f) return INFINITY;
  const float n = rintf(x * 1.44269504088896341f);
  float r = fmaf(n, -0.693145751953125f, x);
  r = fmaf(n, -1.42860682030941723212e-6f, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

/* log of a positive normal x: x = m 2^e, m in [sqrt(1/2), sqrt(2)),
 * log m = 2 atanh(s) with s = (m-1)/(m+1), odd series to s^9. */
float eo_log(float x) {
  int e;
  float m = frexpf(x, &e);
  if (m < 0.70710678118654752f) {
    m = m + m;
    e = e - 1;
  }
  const float f = m - 1.0f;
  const float s = f / (2.0f + f);
  const float z = s * s;
  float p = 2.0f / 9.0f;
  p = fmaf(p, z, 2.0f / 7.0f);
  p = fmaf(p, z, 2.0f / 5.0f);
  p = fmaf(p, z, 2.0f / 3.0f);
  p = fmaf(p, z, 2.0f);
  const float lm = s * p;
  const float ef = (float)e;
  return fmaf(ef, 0.693145751953125f, fmaf(ef, 1.42860682030941723212e-6f, lm));
}

/* sin/cos of an fp32 angle: quadrant reduction in double precision, Taylor
 * polynomials (sin to r^9, cos to r^10) on |r| <= pi/4 in fp32. */
void eo_sincos(float x, float* sn, float* cs) {
  const double xd = (double)x;
  const double kd = rint(xd * 0.63661977236758134308);
  double rd = fma(-kd, 1.5707963267948966192, xd);
  rd = fma(-kd, 6.123233995736766036e-17, rd);
  const float r = (float)rd;
  const float z = r * r;
  float sp = 1.0f / 362880.0f;
  sp = fmaf(sp, z, -1.0f / 5040.0f);
  sp = fmaf(sp, z, 1.0f / 120.0f);
  sp = fmaf(sp, z, -1.0f / 6.0f);
  const float sr = fmaf(sp * z, r, r);
  float cp = -1.0f / 3628800.0f;
  cp = fmaf(cp, z, 1.0f / 40320.0f);
  cp = fmaf(cp, z, -1.0f / 720.0f);
  cp = fmaf(cp, z, 1.0f / 24.0f);
  cp = fmaf(cp, z, -0.5f);
  const float cr = fmaf(cp, z, 1.0f);
  const int q = (int)((long long)kd & 3);
  *sn = q == 0 ? sr : q == 1 ? cr : q == 2 ? -sr : -cr;
  *cs = q == 0 ? cr : q == 1 ? -sr : q == 2 ? -cr : sr;
}

/* MLX unary sigmoid with bf16 boundaries after exp, add, reciprocal and the
 * positive-branch subtraction: linear.metal:389-395, gdn.metal:10-15. */
float eo_sigmoid_bf(float x) {
  float e = BF(eo_exp(fabsf(x)));
  float d = BF(1.0f + e);
  float p = BF(1.0f / d);
  return BF(x < 0.0f ? p : 1.0f - p);
}

/* MLX utils.h log1p specialised to [0,1], gdn.metal:19-23 */
static float mlx_log1p(float x) {
  float xp1 = 1.0f + x;
  if (xp1 == 1.0f) return x;
  return x * (eo_log(xp1) / (xp1 - 1.0f));
}

/* gdn.metal:25-29 */
float eo_softplus_bf(float x) {
  float e = BF(eo_exp(-fabsf(x)));
  float l = BF(mlx_log1p(e));
  return BF(fmaxf(x, 0.0f) + l);
}

/* attention.metal:62-63: exp2(-(pair/32) * log2(1e7)), the exponent formed in
 * fp32 exactly as written and exp2 evaluated accurately (rounded once). */
float eo_rope_inv_freq(int pair) {
  float t = -((float)pair / 32.0f) * 23.253496170043945f;
  return (float)exp2((double)t);
}

/* Pairwise tree in lane order: ((v0+v1)+(v2+v3)) + ... for n a power of two.
 * The reference sums across SIMD lanes with simd_sum, whose order Metal does
 * not specify; this tree is the order the kernels use. Destroys v. */
static float tree(float* v, int n) {
  for (int off = 1; off < n; off *= 2)
    for (int i = 0; i + off < n; i += 2 * off) v[i] = v[i] + v[i + off];
  return v[0];
}

int eo_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
void eo_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------------------------ */
/* linear                                                              */
/* ------------------------------------------------------------------ */
/* embedding_q4, linear.metal:11-24: bf16(scale*q + bias) */
void eo_embedding(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases,
                  int K, uint32_t token, uint16_t* out) {
  for (int k = 0; k < K; ++k) {
    uint32_t q = (codes[(size_t)token * (K / 8) + k / 8] >> (4 * (k % 8))) & 15u;
    size_t g = (size_t)token * (K / 64) + k / 64;
    out[k] = eo_f32_to_bf16(fmaf(F(scales[g]), (float)q, F(biases[g])));
  }
}

/* One output row of the Q4 matvec (linear.metal:38-72 arithmetic: affine
 * dequant s*q + b folded as s*sum(q x) + b*sum(x) per group, fp32, one bf16
 * round). Fixed order: the row is cut into 32-element slices (half a group);
 * per slice xs = sequential sum of x, dot = (fma chain over the even
 * elements) + (fma chain over the odd elements), partial = fma(xs, b, s*dot).
 * K = 1024: tree over the 32 slice partials; K = 2048: tree over 64;
 * other K (<= 4096): lane l holds slice l, adds slice l+64 when present, tree
 * over 64 lanes. */
static float slice_partial(const uint32_t* w, const uint16_t* s, const uint16_t* b, int K,
                           const float* xf, size_t row, int slice) {
  const uint32_t* c = w + row * (size_t)(K / 8) + (size_t)slice * 4;
  const float* x = xf + slice * 32;
  float xs = 0.0f, a0 = 0.0f, a1 = 0.0f;
  for (int j = 0; j < 32; ++j) xs = xs + x[j];
  for (int j = 0; j < 32; ++j) {
    const float q = (float)((c[j / 8] >> (4 * (j % 8))) & 15u);
    if (j & 1) a1 = fmaf(x[j], q, a1);
    else a0 = fmaf(x[j], q, a0);
  }
  const size_t gi = row * (size_t)(K / 64) + slice / 2;
  return fmaf(xs, F(b[gi]), F(s[gi]) * (a0 + a1));
}

static float qmv_row(const uint32_t* w, const uint16_t* s, const uint16_t* b, int K,
                     const float* xf, size_t row) {
  float lane[64];
  const int ns = K / 32;
  if (K == 1024) {
    for (int l = 0; l < 32; ++l) lane[l] = slice_partial(w, s, b, K, xf, row, l);
    return tree(lane, 32);
  }
  for (int l = 0; l < 64; ++l) {
    float p = l < ns ? slice_partial(w, s, b, K, xf, row, l) : 0.0f;
    if (l + 64 < ns) p = p + slice_partial(w, s, b, K, xf, row, l + 64);
    lane[l] = p;
  }
  return tree(lane, 64);
}

void eo_q4_matvec(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases,
                  int N, int K, const uint16_t* x, uint16_t* y, float* y_f32) {
  float* xf = (float*)malloc(sizeof(float) * K);
  eo_bf16_to_f32_array(x, xf, K);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    float v = qmv_row(codes, scales, biases, K, xf, (size_t)n);
    if (y) y[n] = eo_f32_to_bf16(v);
    if (y_f32) y_f32[n] = v;
  }
  free(xf);
}

/* qmv_add_q4, linear.metal:119-122 */
void eo_q4_matvec_add(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases,
                      int N, int K, const uint16_t* x, const uint16_t* residual, uint16_t* y) {
  float* xf = (float*)malloc(sizeof(float) * K);
  eo_bf16_to_f32_array(x, xf, K);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    float v = qmv_row(codes, scales, biases, K, xf, (size_t)n);
    y[n] = eo_f32_to_bf16(F(residual[n]) + BF(v));
  }
  free(xf);
}

/* rms_norm_bf16 arithmetic (linear.metal:311-330): fp32 sum of squares,
 * inv = 1/sqrt(mean + eps), out = bf16(bf16(x*inv)*gain). Fixed order for the
 * 1024-wide rows: 32 slices of 32 (fma chain of squares each), tree over the
 * 32 slice sums. */
void eo_rms_norm(const uint16_t* x, const uint16_t* gain, int cols, float eps, uint16_t* out) {
  float lane[32];
  for (int l = 0; l < 32; ++l) {
    float ss = 0.0f;
    for (int j = 0; j < 32; ++j) {
      int c = l * 32 + j;
      float v = c < cols ? F(x[c]) : 0.0f;
      ss = fmaf(v, v, ss);
    }
    lane[l] = ss;
  }
  float total = tree(lane, 32);
  float inv = 1.0f / sqrtf(total / (float)cols + eps);
  for (int c = 0; c < cols; ++c) out[c] = eo_f32_to_bf16(BF(F(x[c]) * inv) * F(gain[c]));
}

/* swiglu_bf16, linear.metal:388-395 */
void eo_swiglu(const uint16_t* gate, const uint16_t* up, int n, uint16_t* out) {
#pragma omp parallel for schedule(static) if (n > 65536)
  for (int i = 0; i < n; ++i) {
    float g = F(gate[i]);
    float s = eo_sigmoid_bf(g);
    float silu = BF(g * s);
    out[i] = eo_f32_to_bf16(silu * F(up[i]));
  }
}

/* ------------------------------------------------------------------ */
/* Gated DeltaNet                                                      */
/* ------------------------------------------------------------------ */
/* Convolution, SiLU and (for Q and K) normalisation of the 128 channels of
 * one (block, head) group for one token; the group's history channels are
 * touched by no other group. */
static void gdn_conv_group(const uint16_t* raw, uint16_t* history, const uint16_t* conv_w,
                           int block, int h, uint16_t* conv_out) {
  const float q_scale = 0.0078125f;
  const float k_scale = BF(0.08838834764831845f);
  float v[128];
  for (int d = 0; d < 128; ++d) {
    int c = block * 2048 + h * 128 + d;
    uint16_t old0 = history[c], old1 = history[6144 + c], old2 = history[12288 + c];
    float acc = 0.0f;
    acc = fmaf(F(old0), F(conv_w[c * 4 + 0]), acc);
    acc = fmaf(F(old1), F(conv_w[c * 4 + 1]), acc);
    acc = fmaf(F(old2), F(conv_w[c * 4 + 2]), acc);
    acc = fmaf(F(raw[c]), F(conv_w[c * 4 + 3]), acc);
    float xr = BF(acc);
    v[d] = BF(xr * eo_sigmoid_bf(xr));
    history[c] = old1;
    history[6144 + c] = old2;
    history[12288 + c] = raw[c];
  }
  if (block < 2) {
    /* sum of squares: tree over channels 0..63 plus tree over 64..127 */
    float sq[128];
    for (int d = 0; d < 128; ++d) sq[d] = v[d] * v[d];
    float ss = tree(sq, 64) + tree(sq + 64, 64);
    float inv = 1.0f / sqrtf(ss / 128.0f + 1.0e-6f / 128.0f);
    float scale = block == 0 ? q_scale : k_scale;
    for (int d = 0; d < 128; ++d)
      conv_out[block * 2048 + h * 128 + d] = eo_f32_to_bf16(BF(v[d] * inv) * scale);
  } else {
    for (int d = 0; d < 128; ++d) conv_out[block * 2048 + h * 128 + d] = eo_f32_to_bf16(v[d]);
  }
}

static void gdn_gates(const uint16_t* a, const uint16_t* b, const float* a_log,
                      const uint16_t* dt_bias, float* g, uint16_t* beta) {
  for (int h = 0; h < 16; ++h) {
    float ax = BF(F(a[h]) + F(dt_bias[h]));
    g[h] = eo_exp(-eo_exp(a_log[h]) * eo_softplus_bf(ax));
    beta[h] = eo_f32_to_bf16(eo_sigmoid_bf(F(b[h])));
  }
}

void eo_gdn_conv_prepare(const uint16_t* raw, uint16_t* history, const uint16_t* conv_w,
                         const uint16_t* a, const uint16_t* b, const float* a_log,
                         const uint16_t* dt_bias, uint16_t* conv_out, float* g, uint16_t* beta) {
  for (int block = 0; block < 3; ++block)
    for (int h = 0; h < 16; ++h) gdn_conv_group(raw, history, conv_w, block, h, conv_out);
  gdn_gates(a, b, a_log, dt_bias, g, beta);
}

/* gdn_recur, gdn.metal:185-227 with T=1: decay, memory = S.k, delta =
 * (v - memory)*beta, S += k*delta, readout = S.q; fp32 state. Fixed order: a
 * value row is 16 lanes of 8 keys; memory and readout are fma chains over the
 * lane's 8 keys and a tree over the 16 lanes. */
/* One token's update of value row `row` of head h (the state row st). */
static uint16_t gdn_recur_row(const uint16_t* conv, float gt, float bt, int h, int row, float* st) {
  const uint16_t* qv = conv + h * 128;
  const uint16_t* kv = conv + 2048 + h * 128;
  float vv = F(conv[4096 + h * 128 + row]);
  float lane[16];
  for (int j = 0; j < 16; ++j) {
    float acc = 0.0f;
    for (int i = 0; i < 8; ++i) {
      int e = 8 * j + i;
      st[e] = st[e] * gt;
      acc = fmaf(st[e], F(kv[e]), acc);
    }
    lane[j] = acc;
  }
  float memory = tree(lane, 16);
  float delta = (vv - memory) * bt;
  for (int j = 0; j < 16; ++j) {
    float acc = 0.0f;
    for (int i = 0; i < 8; ++i) {
      int e = 8 * j + i;
      st[e] = fmaf(F(kv[e]), delta, st[e]);
      acc = fmaf(st[e], F(qv[e]), acc);
    }
    lane[j] = acc;
  }
  return eo_f32_to_bf16(tree(lane, 16));
}

void eo_gdn_recur(const uint16_t* conv, const float* g, const uint16_t* beta,
                  float* state, uint16_t* y) {
#pragma omp parallel for schedule(static)
  for (int hr = 0; hr < 16 * 128; ++hr) {
    int h = hr / 128, row = hr % 128;
    y[h * 128 + row] = gdn_recur_row(conv, g[h], F(beta[h]), h, row, state + (size_t)hr * 128);
  }
}

/* A state row sees only its own value element and the head's shared q, k,
 * g, beta, so the token loop runs inside the row loop with the same updates
 * in the same order as T calls of eo_gdn_recur. */
void eo_gdn_recur_rows(const uint16_t* conv, const float* g, const uint16_t* beta, int T,
                       float* state, uint16_t* y) {
#pragma omp parallel for schedule(static)
  for (int hr = 0; hr < 16 * 128; ++hr) {
    int h = hr / 128, row = hr % 128;
    for (int t = 0; t < T; ++t)
      y[(size_t)t * 2048 + h * 128 + row] =
          gdn_recur_row(conv + (size_t)t * 6144, g[t * 16 + h], F(beta[t * 16 + h]), h, row,
                        state + (size_t)hr * 128);
  }
}

void eo_gdn_conv_prepare_rows(const uint16_t* raw, uint16_t* history, const uint16_t* conv_w,
                              const uint16_t* a, const uint16_t* b, const float* a_log,
                              const uint16_t* dt_bias, int T, uint16_t* conv_out, float* g,
                              uint16_t* beta) {
  /* a group's channels and history evolve on their own, so each group runs
   * its tokens in order, groups in parallel */
#pragma omp parallel for schedule(static)
  for (int grp = 0; grp < 48; ++grp)
    for (int t = 0; t < T; ++t)
      gdn_conv_group(raw + (size_t)t * 6144, history, conv_w, grp / 16, grp % 16,
                     conv_out + (size_t)t * 6144);
  for (int t = 0; t < T; ++t)
    gdn_gates(a + t * 16, b + t * 16, a_log, dt_bias, g + t * 16, beta + t * 16);
}

void eo_gdn_norm_gate_rows(const uint16_t* y, const uint16_t* z, const uint16_t* w, int T,
                           uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t)
    eo_gdn_norm_gate(y + (size_t)t * 2048, z + (size_t)t * 2048, w, out + (size_t)t * 2048);
}

/* gdn_norm_gate, gdn.metal:238-254 (fp32 sigmoid, unlike the MLX unary one).
 * Fixed order: 16 lanes of 8 channels per head, fma chain of squares, tree
 * over the 16 lanes. */
void eo_gdn_norm_gate(const uint16_t* y, const uint16_t* z, const uint16_t* w, uint16_t* out) {
  for (int h = 0; h < 16; ++h) {
    float lane[16];
    for (int j = 0; j < 16; ++j) {
      float ss = 0.0f;
      for (int i = 0; i < 8; ++i) {
        float v = F(y[h * 128 + 8 * j + i]);
        ss = fmaf(v, v, ss);
      }
      lane[j] = ss;
    }
    float ss = tree(lane, 16);
    float inv = 1.0f / sqrtf(ss / 128.0f + 1.0e-6f);
    for (int d = 0; d < 128; ++d) {
      int off = h * 128 + d;
      float norm = BF(BF(F(y[off]) * inv) * F(w[d]));
      float gate = F(z[off]);
      float sy = 1.0f / (1.0f + eo_exp(fabsf(gate)));
      float sig = gate < 0.0f ? sy : 1.0f - sy;
      out[off] = eo_f32_to_bf16((gate * sig) * norm);
    }
  }
}

/* ------------------------------------------------------------------ */
/* attention                                                           */
/* ------------------------------------------------------------------ */
/* attention.metal:36-53 arithmetic; fixed order: 64 lanes of 4 dims, fma
 * chain of squares, tree over the 64 lanes. */
static float head_inv_rms(const uint16_t* x) {
  float lane[64];
  for (int t = 0; t < 64; ++t) {
    float s = 0.0f;
    for (int i = 0; i < 4; ++i) {
      float v = F(x[4 * t + i]);
      s = fmaf(v, v, s);
    }
    lane[t] = s;
  }
  return 1.0f / sqrtf(tree(lane, 64) / 256.0f + 1e-6f);
}

/* attention.metal:55-70: pairs (i, i+32) for i < 32, angle = pos*inv_freq;
 * d < 32: fma(lo, c, -(hi*s)); 32 <= d < 64: fma(lo, s, hi*c). */
static uint16_t rope_component(const float* normalized, int d, int position) {
  if (d >= 64) return eo_f32_to_bf16(normalized[d]);
  int pair = d % 32;
  float inv_freq = eo_rope_inv_freq(pair);
  float angle = (float)position * inv_freq;
  float s, c;
  eo_sincos(angle, &s, &c);
  float lo = normalized[pair], hi = normalized[pair + 32];
  return eo_f32_to_bf16(d < 32 ? fmaf(lo, c, -(hi * s)) : fmaf(lo, s, hi * c));
}

void eo_attn_prepare(const uint16_t* q_proj, const uint16_t* k, const uint16_t* v,
                     const uint16_t* q_gain, const uint16_t* k_gain, uint16_t* query,
                     uint16_t* kcache, uint16_t* vcache, int position, int capacity) {
  float normalized[256];
  for (int head = 0; head < 8; ++head) {
    const uint16_t* x = q_proj + head * 512;
    float inv = head_inv_rms(x);
    for (int d = 0; d < 256; ++d) normalized[d] = BF(BF(F(x[d]) * inv) * F(q_gain[d]));
    for (int d = 0; d < 256; ++d) query[head * 256 + d] = rope_component(normalized, d, position);
  }
  for (int head = 0; head < 2; ++head) {
    const uint16_t* x = k + head * 256;
    const uint16_t* vv = v + head * 256;
    size_t ci = ((size_t)head * capacity + position) * 256;
    float inv = head_inv_rms(x);
    for (int d = 0; d < 256; ++d) {
      normalized[d] = BF(BF(F(x[d]) * inv) * F(k_gain[d]));
      vcache[ci + d] = vv[d];
    }
    for (int d = 0; d < 256; ++d) kcache[ci + d] = rope_component(normalized, d, position);
  }
}

/* One score, attention_decode.metal:137-144 / 321-326 (q . k with q = k-scale
 * 1/16 times the bf16 query). Fixed order: partial l (0..31) covers dims
 * 8l..8l+7 as an fma chain; lane m (0..7) adds its partials as
 * (p[m] + p[m+8]) + (p[m+16] + p[m+24]); the 8 lane values are added
 * pairwise in lane order. */
static float score_row(const float* q, const uint16_t* krow) {
  float p[32], a[8];
  for (int l = 0; l < 32; ++l) {
    float s = 0.0f;
    for (int j = 0; j < 8; ++j) s = fmaf(q[8 * l + j], F(krow[8 * l + j]), s);
    p[l] = s;
  }
  for (int m = 0; m < 8; ++m) a[m] = (p[m] + p[m + 8]) + (p[m + 16] + p[m + 24]);
  return tree(a, 8);
}

/* One online-softmax update of a position chain (attention_decode.metal:146-157,
 * 328-338): new max, factor and exp score, then sum = sum*factor + e and
 * o = fma(e, v, o*factor). */
static void chain_step(float score, const uint16_t* vrow, float* max_score, float* sum_exp,
                       float* o) {
  float new_max = fmaxf(*max_score, score);
  float factor = eo_exp(*max_score - new_max);
  float es = eo_exp(score - new_max);
  *max_score = new_max;
  *sum_exp = *sum_exp * factor + es;
  for (int d = 0; d < 256; ++d) o[d] = fmaf(es, F(vrow[d]), o[d] * factor);
}

/* sdpa_vector<bf16,256>, attention_decode.metal:51-213: chain sg (0..31) takes
 * positions sg, sg+32, ... in order; chains are combined with factors
 * exp(max_sg - max), sums and outputs added pairwise over the 32 chains. */
void eo_attn_decode_single(const uint16_t* query, const uint16_t* kcache, const uint16_t* vcache,
                           int length, int capacity, uint16_t* out) {
  const float finite_min = -FLT_MAX;
#pragma omp parallel for schedule(static)
  for (int h = 0; h < 8; ++h) {
    int kvh = h / 4;
    float q[256];
    for (int d = 0; d < 256; ++d) q[d] = 0.0625f * F(query[h * 256 + d]);
    const uint16_t* kb = kcache + (size_t)kvh * capacity * 256;
    const uint16_t* vb = vcache + (size_t)kvh * capacity * 256;
    static __thread float o[32][256];
    float mx[32], sm[32];
    for (int sg = 0; sg < 32; ++sg) {
      float max_score = finite_min, sum_exp = 0.0f;
      for (int d = 0; d < 256; ++d) o[sg][d] = 0.0f;
      for (int i = sg; i < length; i += 32)
        chain_step(score_row(q, kb + (size_t)i * 256), vb + (size_t)i * 256, &max_score,
                   &sum_exp, o[sg]);
      mx[sg] = max_score;
      sm[sg] = sum_exp;
    }
    float new_max = mx[0];
    for (int s = 1; s < 32; ++s) new_max = fmaxf(new_max, mx[s]);
    float fac[32], tmp[32];
    for (int s = 0; s < 32; ++s) {
      fac[s] = eo_exp(mx[s] - new_max);
      tmp[s] = sm[s] * fac[s];
    }
    float sum_exp = tree(tmp, 32);
    for (int d = 0; d < 256; ++d) {
      for (int s = 0; s < 32; ++s) tmp[s] = o[s][d] * fac[s];
      float v = tree(tmp, 32);
      v = sum_exp == 0.0f ? v : v / sum_exp;
      out[h * 256 + d] = eo_f32_to_bf16(v);
    }
  }
}

/* sdpa_vector_2pass_1<bf16,256>, attention_decode.metal:215-431, blocks=64:
 * block b takes positions b, b+64, ... in order; unnormalised o rounded to bf16. */
void eo_attn_decode_split(const uint16_t* query, const uint16_t* kcache, const uint16_t* vcache,
                          int length, int capacity, uint16_t* partials, float* sums, float* maxs) {
  const float finite_min = -FLT_MAX;
#pragma omp parallel for schedule(static)
  for (int hb = 0; hb < 8 * 64; ++hb) {
    int h = hb / 64, blk = hb % 64;
    int kvh = h / 4;
    float q[256], o[256];
    for (int d = 0; d < 256; ++d) {
      q[d] = 0.0625f * F(query[h * 256 + d]);
      o[d] = 0.0f;
    }
    const uint16_t* kb = kcache + (size_t)kvh * capacity * 256;
    const uint16_t* vb = vcache + (size_t)kvh * capacity * 256;
    float max_score = finite_min, sum_exp = 0.0f;
    for (int i = blk; i < length; i += 64)
      chain_step(score_row(q, kb + (size_t)i * 256), vb + (size_t)i * 256, &max_score, &sum_exp,
                 o);
    sums[h * 64 + blk] = sum_exp;
    maxs[h * 64 + blk] = max_score;
    for (int d = 0; d < 256; ++d) partials[((size_t)h * 64 + blk) * 256 + d] = eo_f32_to_bf16(o[d]);
  }
}

/* attn_decode_split2_gate, attention_decode.metal:841-890 */
void eo_attn_split_merge_gate(const uint16_t* partials, const float* sums, const float* maxs,
                              const uint16_t* q_proj, uint16_t* gated) {
  for (int h = 0; h < 8; ++h) {
    const float* hs = sums + h * 64;
    const float* hm = maxs + h * 64;
    float M = -FLT_MAX;
    for (int b = 0; b < 64; ++b) M = fmaxf(M, hm[b]);
    float lane[32];
    for (int l = 0; l < 32; ++l) {
      float s = 0.0f;
      for (int bb = 0; bb < 2; ++bb) s += eo_exp(hm[l + 32 * bb] - M) * hs[l + 32 * bb];
      lane[l] = s;
    }
    float sum_exp = tree(lane, 32);
    for (int d = 0; d < 256; ++d) {
      for (int l = 0; l < 32; ++l) {
        float o = 0.0f;
        for (int bb = 0; bb < 2; ++bb) {
          int b = l + 32 * bb;
          o += eo_exp(hm[b] - M) * F(partials[((size_t)h * 64 + b) * 256 + d]);
        }
        lane[l] = o;
      }
      float o = tree(lane, 32);
      o = sum_exp == 0.0f ? o : o / sum_exp;
      float attention = BF(o);
      float gate = eo_sigmoid_bf(F(q_proj[h * 512 + 256 + d]));
      gated[h * 256 + d] = eo_f32_to_bf16(attention * gate);
    }
  }
}

/* attn_gate, attention.metal:140-150 */
void eo_attn_gate(const uint16_t* attn, const uint16_t* q_proj, uint16_t* gated) {
  for (int i = 0; i < 2048; ++i) {
    int head = i / 256, d = i % 256;
    float gate = eo_sigmoid_bf(F(q_proj[head * 512 + 256 + d]));
    gated[i] = eo_f32_to_bf16(F(attn[i]) * gate);
  }
}

/* model.rs:327-347 */
void eo_attn_decode_gated(const uint16_t* query, const uint16_t* kcache, const uint16_t* vcache,
                          int length, int capacity, const uint16_t* q_proj, uint16_t* gated) {
  if (length < 1024) {
    uint16_t o[2048];
    eo_attn_decode_single(query, kcache, vcache, length, capacity, o);
    eo_attn_gate(o, q_proj, gated);
  } else {
    uint16_t* partials = (uint16_t*)malloc(sizeof(uint16_t) * 8 * 64 * 256);
    float sums[8 * 64], maxs[8 * 64];
    eo_attn_decode_split(query, kcache, vcache, length, capacity, partials, sums, maxs);
    eo_attn_split_merge_gate(partials, sums, maxs, q_proj, gated);
    free(partials);
  }
}

/* ------------------------------------------------------------------ */
/* head                                                                */
/* ------------------------------------------------------------------ */
/* head_lse_g8 + head_lse_tail arithmetic (head_lse.metal:51-97): logits are
 * bf16; lse = bf16(log(sum exp(l - max)) + max); token = lowest index of the
 * maximum of bf16(l - lse) (docs/protocol.md:44). Fixed order: blocks of 256
 * consecutive logits, block max exact, block sum = (w0 + w1) + (w2 + w3) where
 * w is a tree over a 64-logit quarter of exp(l - blockmax) (0 past the end);
 * the global sum has 256 accumulators, accumulator t adding
 * sum_b * exp(max_b - max) for blocks b = t, t+256, ... in order, then the
 * same 4 x 64 tree-and-pairs combination. */
uint32_t eo_greedy(const uint16_t* logits, int n, float* lse_out) {
  const int nb = (n + 255) / 256;
  float* pmax = (float*)malloc(sizeof(float) * nb);
  float* psum = (float*)malloc(sizeof(float) * nb);
  for (int b = 0; b < nb; ++b) {
    float m = -INFINITY;
    for (int i = 0; i < 256; ++i)
      if (b * 256 + i < n) m = fmaxf(m, F(logits[b * 256 + i]));
    float w[4];
    for (int q = 0; q < 4; ++q) {
      float e[64];
      for (int i = 0; i < 64; ++i) {
        int r = b * 256 + q * 64 + i;
        e[i] = r < n ? eo_exp(F(logits[r]) - m) : 0.0f;
      }
      w[q] = tree(e, 64);
    }
    pmax[b] = m;
    psum[b] = (w[0] + w[1]) + (w[2] + w[3]);
  }
  float gm = -FLT_MAX;
  for (int b = 0; b < nb; ++b) gm = fmaxf(gm, pmax[b]);
  float acc[256];
  for (int t = 0; t < 256; ++t) {
    float a = 0.0f;
    for (int b = t; b < nb; b += 256) a = a + psum[b] * eo_exp(pmax[b] - gm);
    acc[t] = a;
  }
  float w4[4];
  for (int q = 0; q < 4; ++q) w4[q] = tree(acc + 64 * q, 64);
  float gs = (w4[0] + w4[1]) + (w4[2] + w4[3]);
  float lse = BF(eo_log(gs) + gm);
  if (lse_out) *lse_out = lse;
  float target = BF(gm - lse);
  uint32_t id = 0;
  for (int i = 0; i < n; ++i)
    if (BF(F(logits[i]) - lse) == target) {
      id = (uint32_t)i;
      break;
    }
  free(pmax);
  free(psum);
  return id;
}

/* ------------------------------------------------------------------ */
/* full decode step: model.rs:228-307 (rows==1) and :308-350          */
/* ------------------------------------------------------------------ */
static void lin(const eo_linear* L, const uint16_t* x, uint16_t* y) {
  eo_q4_matvec(L->w, L->s, L->b, L->n, L->k, x, y, NULL);
}

uint32_t eo_model_step(const eo_model* m, eo_state* st, uint32_t token, int position,
                       int want_head, uint16_t* logits, uint16_t* hidden_out) {
  uint16_t h[1024], u[1024];
  uint16_t* buf = (uint16_t*)malloc(sizeof(uint16_t) * (6144 + 2048 * 6 + 3584 * 3 + 64));
  uint16_t* qkv = buf;
  uint16_t* z = qkv + 6144;
  uint16_t* conv = z + 2048;         /* 6144 */
  uint16_t* mixed = conv + 6144;     /* 2048 */
  uint16_t* gated = mixed + 2048;    /* 2048 */
  uint16_t* gate = gated + 2048;     /* 3584 */
  uint16_t* up = gate + 3584;        /* 3584 */
  uint16_t* act = up + 3584;         /* 3584 */
  uint16_t* ab = act + 3584;         /* 32 */
  uint16_t beta[16];
  float g[16];
  uint16_t q[4096], kk[512], vv[512], query[2048];

  eo_embedding(m->embed.w, m->embed.s, m->embed.b, 1024, token, h);
  for (int l = 0; l < m->n_layers; ++l) {
    const eo_layer* L = &m->layers[l];
    eo_rms_norm(h, L->input_norm, 1024, 1e-6f, u);
    if (!L->is_attention) {
      lin(&L->qkv, u, qkv);
      lin(&L->z, u, z);
      lin(&L->a, u, ab);
      lin(&L->b, u, ab + 16);
      eo_gdn_conv_prepare(qkv, st->history[l], L->conv_w, ab, ab + 16, L->a_log, L->dt_bias,
                          conv, g, beta);
      eo_gdn_recur(conv, g, beta, st->state[l], mixed);
      eo_gdn_norm_gate(mixed, z, L->gdn_norm, gated);
      eo_q4_matvec_add(L->out.w, L->out.s, L->out.b, 1024, 2048, gated, h, h);
    } else {
      lin(&L->q, u, q);
      lin(&L->k, u, kk);
      lin(&L->v, u, vv);
      eo_attn_prepare(q, kk, vv, L->q_norm, L->k_norm, query, st->kcache[l], st->vcache[l],
                      position, st->capacity);
      eo_attn_decode_gated(query, st->kcache[l], st->vcache[l], position + 1, st->capacity, q,
                           gated);
      eo_q4_matvec_add(L->o.w, L->o.s, L->o.b, 1024, 2048, gated, h, h);
    }
    eo_rms_norm(h, L->post_norm, 1024, 1e-6f, u);
    lin(&L->gate, u, gate);
    lin(&L->up, u, up);
    eo_swiglu(gate, up, 3584, act);
    eo_q4_matvec_add(L->down.w, L->down.s, L->down.b, 1024, 3584, act, h, h);
  }
  if (hidden_out) memcpy(hidden_out, h, sizeof(h));
  uint32_t tok = 0;
  if (want_head) {
    eo_rms_norm(h, m->final_norm, 1024, 1e-6f, u);
    uint16_t* lg = logits ? logits : (uint16_t*)malloc(sizeof(uint16_t) * (size_t)m->vocab);
    eo_q4_matvec(m->embed.w, m->embed.s, m->embed.b, m->vocab, 1024, u, lg, NULL);
    tok = eo_greedy(lg, m->vocab, NULL);
    if (!logits) free(lg);
  }
  free(buf);
  return tok;
}
