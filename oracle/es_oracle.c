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

/* MLX unary sigmoid with bf16 boundaries after exp, add, reciprocal and the
 * positive-branch subtraction: linear.metal:389-395, gdn.metal:10-15. */
float eo_sigmoid_bf(float x) {
  float e = BF(expf(fabsf(x)));
  float d = BF(1.0f + e);
  float p = BF(1.0f / d);
  return BF(x < 0.0f ? p : 1.0f - p);
}

/* MLX utils.h log1p specialised to [0,1], gdn.metal:19-23 */
static float mlx_log1p(float x) {
  float xp1 = 1.0f + x;
  if (xp1 == 1.0f) return x;
  return x * (logf(xp1) / (xp1 - 1.0f));
}

/* gdn.metal:25-29 */
float eo_softplus_bf(float x) {
  float e = BF(expf(-fabsf(x)));
  float l = BF(mlx_log1p(e));
  return BF(fmaxf(x, 0.0f) + l);
}

/* attention.metal:62-63: exp2(-(pair/32) * log2(1e7)), the exponent formed in
 * fp32 exactly as written and exp2 evaluated accurately (rounded once). */
float eo_rope_inv_freq(int pair) {
  float t = -((float)pair / 32.0f) * 23.253496170043945f;
  return (float)exp2((double)t);
}

/* xor-butterfly restatement of a 2^k-lane simd_sum; destroys v */
static float bfly_sum(float* v, int n) {
  for (int off = n / 2; off >= 1; off /= 2)
    for (int i = 0; i < off; ++i) v[i] = v[i] + v[i + off];
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
    out[k] = eo_f32_to_bf16(F(scales[g]) * (float)q + F(biases[g]));
  }
}

/* One output row of qmv_q4, linear.metal:38-72: 32 lanes, each a 16-wide K
 * slice per 512-block; lane partial s*dot + xs*b accumulated over blocks. */
static float qmv_row(const uint32_t* w, const uint16_t* s, const uint16_t* b, int K,
                     const float* xf, size_t row) {
  float lane_acc[32];
  for (int l = 0; l < 32; ++l) lane_acc[l] = 0.0f;
  const uint16_t* wrow = (const uint16_t*)(w + row * (size_t)(K / 8));
  for (int k0 = 0; k0 < K; k0 += 512) {
    for (int lane = 0; lane < 32; ++lane) {
      int k = k0 + lane * 16;
      float xx[16];
      float xs = 0.0f;
      for (int j = 0; j < 16; j += 4) {
        float a = xf[k + j], bb = xf[k + j + 1], c = xf[k + j + 2], d = xf[k + j + 3];
        xs += ((a + bb) + c) + d;
        xx[j] = a;
        xx[j + 1] = bb / 16.0f;
        xx[j + 2] = c / 256.0f;
        xx[j + 3] = d / 4096.0f;
      }
      const uint16_t* ww = wrow + k / 4;
      float dotq = 0.0f;
      for (int j = 0; j < 4; ++j) {
        uint16_t v = ww[j];
        dotq += ((xx[4 * j] * (float)(v & 0x000f) + xx[4 * j + 1] * (float)(v & 0x00f0)) +
                 xx[4 * j + 2] * (float)(v & 0x0f00)) +
                xx[4 * j + 3] * (float)(v & 0xf000);
      }
      size_t gi = row * (size_t)(K / 64) + k / 64;
      lane_acc[lane] += F(s[gi]) * dotq + xs * F(b[gi]);
    }
  }
  return bfly_sum(lane_acc, 32);
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

/* rms_norm_bf16, linear.metal:311-330: four contiguous values per thread,
 * simd_sum per 32 threads, then a simd_sum over the group partials. */
void eo_rms_norm(const uint16_t* x, const uint16_t* gain, int cols, float eps, uint16_t* out) {
  int threads = ((cols + 127) / 128) * 32;
  int sgs = threads / 32;
  float sums[32];
  for (int i = 0; i < 32; ++i) sums[i] = 0.0f;
  for (int sg = 0; sg < sgs; ++sg) {
    float lane[32];
    for (int l = 0; l < 32; ++l) {
      int t = sg * 32 + l;
      float acc = 0.0f;
      for (int j = 0; j < 4; ++j) {
        int c = t * 4 + j;
        float v = c < cols ? F(x[c]) : 0.0f;
        acc += v * v;
      }
      lane[l] = acc;
    }
    sums[sg] = bfly_sum(lane, 32);
  }
  float total = bfly_sum(sums, 32);
  float inv = 1.0f / sqrtf(total / (float)cols + eps);
  for (int c = 0; c < cols; ++c) out[c] = eo_f32_to_bf16(BF(F(x[c]) * inv) * F(gain[c]));
}

/* swiglu_bf16, linear.metal:388-395 */
void eo_swiglu(const uint16_t* gate, const uint16_t* up, int n, uint16_t* out) {
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
void eo_gdn_conv_prepare(const uint16_t* raw, uint16_t* history, const uint16_t* conv_w,
                         const uint16_t* a, const uint16_t* b, const float* a_log,
                         const uint16_t* dt_bias, uint16_t* conv_out, float* g, uint16_t* beta) {
  const float q_scale = 0.0078125f;
  const float k_scale = BF(0.08838834764831845f);
  for (int block = 0; block < 3; ++block) {
    for (int h = 0; h < 16; ++h) {
      float v[32][4];
      float lane_ss[32];
      for (int lane = 0; lane < 32; ++lane) {
        int off = block * 2048 + h * 128 + lane * 4;
        float ss = 0.0f;
        for (int i = 0; i < 4; ++i) {
          int c = off + i;
          uint16_t old0 = history[c], old1 = history[6144 + c], old2 = history[12288 + c];
          float acc = 0.0f;
          for (int tap = 0; tap < 4; ++tap) {
            float xv = tap == 0 ? F(old0) : tap == 1 ? F(old1) : tap == 2 ? F(old2) : F(raw[c]);
            acc = fmaf(xv, F(conv_w[c * 4 + tap]), acc);
          }
          float xr = BF(acc);
          v[lane][i] = BF(xr * eo_sigmoid_bf(xr));
          ss += v[lane][i] * v[lane][i];
          history[c] = old1;
          history[6144 + c] = old2;
          history[12288 + c] = raw[c];
        }
        lane_ss[lane] = ss;
      }
      if (block < 2) {
        float ss = bfly_sum(lane_ss, 32);
        float inv = 1.0f / sqrtf(ss / 128.0f + 1.0e-6f / 128.0f);
        float scale = block == 0 ? q_scale : k_scale;
        for (int lane = 0; lane < 32; ++lane)
          for (int i = 0; i < 4; ++i)
            conv_out[block * 2048 + h * 128 + lane * 4 + i] =
                eo_f32_to_bf16(BF(v[lane][i] * inv) * scale);
      } else {
        for (int lane = 0; lane < 32; ++lane)
          for (int i = 0; i < 4; ++i)
            conv_out[block * 2048 + h * 128 + lane * 4 + i] = eo_f32_to_bf16(v[lane][i]);
      }
    }
  }
  for (int h = 0; h < 16; ++h) {
    float ax = BF(F(a[h]) + F(dt_bias[h]));
    g[h] = expf(-expf(a_log[h]) * eo_softplus_bf(ax));
    beta[h] = eo_f32_to_bf16(eo_sigmoid_bf(F(b[h])));
  }
}

/* gdn_recur, gdn.metal:185-227 with T=1. Four lanes own a value row, 32 keys each. */
void eo_gdn_recur(const uint16_t* conv, const float* g, const uint16_t* beta,
                  float* state, uint16_t* y) {
#pragma omp parallel for schedule(static)
  for (int hr = 0; hr < 16 * 128; ++hr) {
    int h = hr / 128, row = hr % 128;
    float gt = g[h];
    float bt = F(beta[h]);
    float mem_l[4], out_l[4];
    float* st = state + ((size_t)h * 128 + row) * 128;
    const uint16_t* qv = conv + h * 128;
    const uint16_t* kv = conv + 2048 + h * 128;
    float vv = F(conv[4096 + h * 128 + row]);
    for (int l = 0; l < 4; ++l) {
      float part[8];
      for (int pb = 0; pb < 8; ++pb) {
        float acc = 0.0f;
        for (int i = 0; i < 4; ++i) {
          int e = l * 32 + pb * 4 + i;
          st[e] = st[e] * gt;
          acc += st[e] * F(kv[e]);
        }
        part[pb] = acc;
      }
      mem_l[l] = ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
    }
    float memory = (mem_l[0] + mem_l[1]) + (mem_l[2] + mem_l[3]);
    float delta = (vv - memory) * bt;
    for (int l = 0; l < 4; ++l) {
      float part[8];
      for (int pb = 0; pb < 8; ++pb) {
        float acc = 0.0f;
        for (int i = 0; i < 4; ++i) {
          int e = l * 32 + pb * 4 + i;
          st[e] = st[e] + F(kv[e]) * delta;
          acc += st[e] * F(qv[e]);
        }
        part[pb] = acc;
      }
      out_l[l] = ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
    }
    float out = (out_l[0] + out_l[1]) + (out_l[2] + out_l[3]);
    y[h * 128 + row] = eo_f32_to_bf16(out);
  }
}

/* gdn_norm_gate, gdn.metal:238-254 (fp32 sigmoid, unlike the MLX unary one) */
void eo_gdn_norm_gate(const uint16_t* y, const uint16_t* z, const uint16_t* w, uint16_t* out) {
  for (int h = 0; h < 16; ++h) {
    float lane_ss[32];
    for (int lane = 0; lane < 32; ++lane) {
      float ss = 0.0f;
      for (int i = 0; i < 4; ++i) {
        float v = F(y[h * 128 + lane * 4 + i]);
        ss += v * v;
      }
      lane_ss[lane] = ss;
    }
    float ss = bfly_sum(lane_ss, 32);
    float inv = 1.0f / sqrtf(ss / 128.0f + 1.0e-6f);
    for (int d = 0; d < 128; ++d) {
      int off = h * 128 + d;
      float norm = BF(BF(F(y[off]) * inv) * F(w[d]));
      float gate = F(z[off]);
      float sy = 1.0f / (1.0f + expf(fabsf(gate)));
      float sig = gate < 0.0f ? sy : 1.0f - sy;
      out[off] = eo_f32_to_bf16((gate * sig) * norm);
    }
  }
}

/* ------------------------------------------------------------------ */
/* attention                                                           */
/* ------------------------------------------------------------------ */
/* attention.metal:36-53: 64 threads x 4 values, two simd sums added */
static float head_inv_rms(const uint16_t* x) {
  float sums[2];
  for (int sg = 0; sg < 2; ++sg) {
    float lane[32];
    for (int l = 0; l < 32; ++l) {
      int t = sg * 32 + l;
      float s = 0.0f;
      for (int i = 0; i < 4; ++i) {
        float v = F(x[4 * t + i]);
        s += v * v;
      }
      lane[l] = s;
    }
    sums[sg] = bfly_sum(lane, 32);
  }
  return 1.0f / sqrtf((sums[0] + sums[1]) / 256.0f + 1e-6f);
}

/* attention.metal:55-70 */
static uint16_t rope_component(const float* normalized, int d, int position) {
  if (d >= 64) return eo_f32_to_bf16(normalized[d]);
  int pair = d % 32;
  float inv_freq = eo_rope_inv_freq(pair);
  float angle = (float)position * inv_freq;
  float c = cosf(angle), s = sinf(angle);
  float lo = normalized[pair], hi = normalized[pair + 32];
  return eo_f32_to_bf16(d < 32 ? lo * c - hi * s : lo * s + hi * c);
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

static float lane_score(const float* q, const uint16_t* krow, int lane) {
  float score = 0.0f;
  for (int j = 0; j < 8; ++j) score += q[lane * 8 + j] * F(krow[lane * 8 + j]);
  return score;
}

static float simd_score(const float* q, const uint16_t* krow) {
  float lanes[32];
  for (int l = 0; l < 32; ++l) lanes[l] = lane_score(q, krow, l);
  return bfly_sum(lanes, 32);
}

/* sdpa_vector<bf16,256>, attention_decode.metal:51-213 (32 simdgroups) */
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
      for (int i = sg; i < length; i += 32) {
        float score = simd_score(q, kb + (size_t)i * 256);
        float new_max = fmaxf(max_score, score);
        float factor = expf(max_score - new_max);
        float es = expf(score - new_max);
        max_score = new_max;
        sum_exp = sum_exp * factor + es;
        for (int d = 0; d < 256; ++d) o[sg][d] = o[sg][d] * factor + es * F(vb[(size_t)i * 256 + d]);
      }
      mx[sg] = max_score;
      sm[sg] = sum_exp;
    }
    float new_max = mx[0];
    for (int s = 1; s < 32; ++s) new_max = fmaxf(new_max, mx[s]);
    float fac[32], tmp[32];
    for (int s = 0; s < 32; ++s) {
      fac[s] = expf(mx[s] - new_max);
      tmp[s] = sm[s] * fac[s];
    }
    float sum_exp = bfly_sum(tmp, 32);
    for (int d = 0; d < 256; ++d) {
      for (int s = 0; s < 32; ++s) tmp[s] = o[s][d] * fac[s];
      float v = bfly_sum(tmp, 32);
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
    for (int i = blk; i < length; i += 64) {
      float score = simd_score(q, kb + (size_t)i * 256);
      float new_max = fmaxf(max_score, score);
      float factor = expf(max_score - new_max);
      float es = expf(score - new_max);
      max_score = new_max;
      sum_exp = sum_exp * factor + es;
      for (int d = 0; d < 256; ++d) o[d] = o[d] * factor + es * F(vb[(size_t)i * 256 + d]);
    }
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
      for (int bb = 0; bb < 2; ++bb) s += expf(hm[l + 32 * bb] - M) * hs[l + 32 * bb];
      lane[l] = s;
    }
    float sum_exp = bfly_sum(lane, 32);
    for (int d = 0; d < 256; ++d) {
      for (int l = 0; l < 32; ++l) {
        float o = 0.0f;
        for (int bb = 0; bb < 2; ++bb) {
          int b = l + 32 * bb;
          o += expf(hm[b] - M) * F(partials[((size_t)h * 64 + b) * 256 + d]);
        }
        lane[l] = o;
      }
      float o = bfly_sum(lane, 32);
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
/* head_lse_g8 (:15-63) online (max,sum) per owner of 4-logit tiles, then
 * head_lse_tail (:66-97): lse = bf16(log(sum)+max); token = lowest index of
 * the maximum of bf16(logit - lse). */
uint32_t eo_greedy(const uint16_t* logits, int n, float* lse_out) {
  float pmax[1024], psum[1024];
  int tiles = (n + 4095) / 4096;
  for (int owner = 0; owner < 1024; ++owner) {
    float vmax = -FLT_MAX, normalizer = 0.0f;
    for (int tile = 0; tile < tiles; ++tile) {
      int row0 = tile * 4096 + owner * 4;
      float vals[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      if (row0 < n)
        for (int q = 0; q < 4; ++q)
          if (row0 + q < n) vals[q] = F(logits[row0 + q]);
      float prev = vmax;
      for (int j = 0; j < 4; ++j) vmax = fmaxf(vmax, vals[j]);
      normalizer *= expf(prev - vmax);
      for (int j = 0; j < 4; ++j) normalizer += expf(vals[j] - vmax);
    }
    pmax[owner] = vmax;
    psum[owner] = normalizer;
  }
  /* tail: 32 simdgroups of 32 */
  float sg_max[32], sg_sum[32];
  for (int sg = 0; sg < 32; ++sg) {
    float m = -FLT_MAX;
    for (int l = 0; l < 32; ++l) m = fmaxf(m, pmax[sg * 32 + l]);
    float lane[32];
    for (int l = 0; l < 32; ++l) lane[l] = psum[sg * 32 + l] * expf(pmax[sg * 32 + l] - m);
    sg_max[sg] = m;
    sg_sum[sg] = bfly_sum(lane, 32);
  }
  float vmax = -FLT_MAX;
  for (int s = 0; s < 32; ++s) vmax = fmaxf(vmax, sg_max[s]);
  float lane[32];
  for (int s = 0; s < 32; ++s) lane[s] = sg_sum[s] * expf(sg_max[s] - vmax);
  float normalizer = bfly_sum(lane, 32);
  float lse = BF(logf(normalizer) + vmax);
  if (lse_out) *lse_out = lse;
  float best = -INFINITY;
  uint32_t id = 0xffffffffu;
  for (int i = 0; i < n; ++i) {
    float v = BF(F(logits[i]) - lse);
    if (v > best) {
      best = v;
      id = (uint32_t)i;
    }
  }
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
