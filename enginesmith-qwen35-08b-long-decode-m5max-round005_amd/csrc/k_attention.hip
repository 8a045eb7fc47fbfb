// Long-context GQA decode attention on gfx950 (8 query heads, 2 KV heads,
// head dim 256, one query token), as a split-K flash decode.
//
// k_attn_split: grid (splits, 2 KV heads), 256 threads. Each block streams a
// contiguous chunk of one KV head's cache exactly once and serves all four
// query heads of that group. A 16-lane row owns one position per step (16
// dims = 32 B of K and of V per lane, 2 positions per pass); scores use
// v_dot2 on bf16 pairs (q is bf16 and q*1/16 is exact), the 16-lane sum is a
// DPP row reduction, and the online softmax keeps fp32 (max, sum, o[256]).
// The 16 row-states of the block are merged in LDS and one fp32 partial per
// (query head, split) is written.
// The prologue fuses attn_prepare_qkv_decode (attention.metal:262-313): q/k
// RMSNorm (eps 1e-6, bf16 normalised value, bf16 gain product) and partial
// RoPE on dims 0..63 with pairs (i, i+32). The block of the last split also
// writes the new K/V row at `position` and scores it from LDS.
//
// k_attn_merge: grid (8 heads, 8 x 32 dims): log-sum-exp merge of the
// partials, then gated = bf16(bf16(o) * sigmoid_bf(gate))
// (attention_decode.metal:841-890, attention.metal:140-150).
#include "es_kernels.hpp"

namespace es {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxSplits = 1024;

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Normalise 4 consecutive dims of a 256-wide head held by a full wave.
__device__ __forceinline__ void head_norm4(const uint16_t* x, const uint16_t* gain, int lane,
                                           float* out) {
  const uint2 xv = *reinterpret_cast<const uint2*>(x + lane * 4);
  const uint2 gv = *reinterpret_cast<const uint2*>(gain + lane * 4);
  const float xf[4] = {bf_lo(xv.x), bf_hi(xv.x), bf_lo(xv.y), bf_hi(xv.y)};
  const float gf[4] = {bf_lo(gv.x), bf_hi(gv.x), bf_lo(gv.y), bf_hi(gv.y)};
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss = fmaf(xf[i], xf[i], ss);
  ss = tree64(ss);
  const float inv = 1.0f / sqrtf(ss / 256.0f + 1e-6f);
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = rbf(rbf(xf[i] * inv) * gf[i]);
}

// Rotary component d of a normalised head (attention.metal:55-70):
// d < 32: fma(lo, c, -(hi*s)); 32 <= d < 64: fma(lo, s, hi*c).
__device__ __forceinline__ float rope_at(const float* nrm, int d, int pos, const float* inv_freq) {
  if (d >= 64) return nrm[d];
  const int pair = d & 31;
  const float angle = (float)pos * inv_freq[pair];
  float s, c;
  es_sincos(angle, &s, &c);
  const float lo = nrm[pair], hi = nrm[pair + 32];
  return rbf(d < 32 ? fmaf(lo, c, -(hi * s)) : fmaf(lo, s, hi * c));
}

// Two consecutive positions of one 16-lane row: 32 B of K and of V each.
struct KvPair {
  u32x4 k0[2], k1[2], v0[2], v1[2];
};

// Load positions p and p+1 when they are below `end`; positions past the end
// are clamped to a valid row and masked by the caller.
__device__ __forceinline__ void kv_load(const uint16_t* kb, const uint16_t* vb, int p, int end,
                                        KvPair& r) {
  const int pa = p < end ? p : 0;
  const int pb = p + 1 < end ? p + 1 : pa;
  const u32x4* k0p = reinterpret_cast<const u32x4*>(kb + (size_t)pa * 256);
  const u32x4* k1p = reinterpret_cast<const u32x4*>(kb + (size_t)pb * 256);
  const u32x4* v0p = reinterpret_cast<const u32x4*>(vb + (size_t)pa * 256);
  const u32x4* v1p = reinterpret_cast<const u32x4*>(vb + (size_t)pb * 256);
  if (p < end) {
    r.k0[0] = k0p[0]; r.k0[1] = k0p[1];
    r.k1[0] = k1p[0]; r.k1[1] = k1p[1];
    r.v0[0] = v0p[0]; r.v0[1] = v0p[1];
    r.v1[0] = v1p[0]; r.v1[1] = v1p[1];
  }
}

__global__ __launch_bounds__(256) void k_attn_split(AttnArgs a) {
  __shared__ float nrm[5][256];           // normalised q heads 0..3, new k
  __shared__ uint32_t qpk[4][128];        // roped q * 1/16, bf16 pairs
  __shared__ uint32_t kvnew[2][128];      // new K (roped) and V rows, bf16 pairs
  __shared__ float mx[16][4];
  __shared__ float osum[4][4][256];
  __shared__ float lsum[4][4];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int g = blockIdx.y, split = blockIdx.x, S = gridDim.x;
  const int pos = load_pos(a.st, a.pos_val);
  const int cached = pos;  // cache rows [0, pos) hold earlier tokens
  int chunk = (cached + S - 1) / S;
  chunk = (chunk + 7) & ~7;
  const int start = min(split * chunk, cached);
  const int end = min(start + chunk, cached);
  const bool last = split == S - 1;

  // First K/V rows of this block's chunk: issued before the prologue so the
  // memory latency overlaps the q normalisation and rotary math.
  const int grp = lane >> 4, j = lane & 15;
  const int G = wave * 4 + grp;  // row-state id 0..15
  const uint16_t* kb = a.kcache + (size_t)g * a.capacity * 256 + j * 16;
  const uint16_t* vb = a.vcache + (size_t)g * a.capacity * 256 + j * 16;
  KvPair cur, nxt;
  int p0 = start + 2 * G;
  kv_load(kb, vb, p0, end, cur);

  // ---- prologue: q (and new k/v for the last split) ----
  {
    float o4[4];
    head_norm4(a.q_proj + (4 * g + wave) * 512, a.q_gain, lane, o4);
#pragma unroll
    for (int i = 0; i < 4; ++i) nrm[wave][lane * 4 + i] = o4[i];
    if (last && wave == 0) {
      head_norm4(a.k_proj + g * 256, a.k_gain, lane, o4);
#pragma unroll
      for (int i = 0; i < 4; ++i) nrm[4][lane * 4 + i] = o4[i];
    }
  }
  __syncthreads();
  {
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = rope_at(nrm[wave], lane * 4 + i, pos, a.inv_freq);
    if (a.query_out && split == 0) {
      uint16_t* qo = a.query_out + (4 * g + wave) * 256 + lane * 4;
      *reinterpret_cast<uint2*>(qo) = make_uint2(pack_bf2(r[0], r[1]), pack_bf2(r[2], r[3]));
    }
    qpk[wave][lane * 2] = pack_bf2(r[0] * 0.0625f, r[1] * 0.0625f);
    qpk[wave][lane * 2 + 1] = pack_bf2(r[2] * 0.0625f, r[3] * 0.0625f);
    if (last && wave == 1) {
      float kr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) kr[i] = rope_at(nrm[4], lane * 4 + i, pos, a.inv_freq);
      const uint32_t k0 = pack_bf2(kr[0], kr[1]);
      const uint32_t k1 = pack_bf2(kr[2], kr[3]);
      kvnew[0][lane * 2] = k0;
      kvnew[0][lane * 2 + 1] = k1;
      const size_t ci = ((size_t)g * a.capacity + pos) * 256 + lane * 4;
      *reinterpret_cast<uint2*>(a.kcache + ci) = make_uint2(k0, k1);
      const uint2 vv = *reinterpret_cast<const uint2*>(a.v_proj + g * 256 + lane * 4);
      kvnew[1][lane * 2] = vv.x;
      kvnew[1][lane * 2 + 1] = vv.y;
      *reinterpret_cast<uint2*>(a.vcache + ci) = vv;
    }
  }
  __syncthreads();

  // ---- main loop ----
  uint32_t q[4][8];
#pragma unroll
  for (int hh = 0; hh < 4; ++hh)
#pragma unroll
    for (int i = 0; i < 8; ++i) q[hh][i] = qpk[hh][j * 8 + i];
  float m[4], l[4], o[4][16];
#pragma unroll
  for (int hh = 0; hh < 4; ++hh) {
    m[hh] = -3.402823466e38f;
    l[hh] = 0.0f;
#pragma unroll
    for (int d = 0; d < 16; ++d) o[hh][d] = 0.0f;
  }
  for (; p0 < end; p0 += 32) {
    kv_load(kb, vb, p0 + 32, end, nxt);
    const bool ok1 = p0 + 1 < end;
    const u32x4 ka0 = cur.k0[0], ka1 = cur.k0[1], kb0 = cur.k1[0], kb1 = cur.k1[1];
    const u32x4 va0 = cur.v0[0], va1 = cur.v0[1], vb0 = cur.v1[0], vb1 = cur.v1[1];
    float s0[4], s1[4];
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      float x0 = 0.0f, x1 = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x0 = dot2(ka0[i], q[hh][i], x0);
        x1 = dot2(kb0[i], q[hh][i], x1);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x0 = dot2(ka1[i], q[hh][4 + i], x0);
        x1 = dot2(kb1[i], q[hh][4 + i], x1);
      }
      s0[hh] = tree16(x0);
      s1[hh] = ok1 ? tree16(x1) : -INFINITY;
    }
    float vf0[16], vf1[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      vf0[2 * i] = bf_lo(va0[i]); vf0[2 * i + 1] = bf_hi(va0[i]);
      vf0[8 + 2 * i] = bf_lo(va1[i]); vf0[8 + 2 * i + 1] = bf_hi(va1[i]);
      vf1[2 * i] = bf_lo(vb0[i]); vf1[2 * i + 1] = bf_hi(vb0[i]);
      vf1[8 + 2 * i] = bf_lo(vb1[i]); vf1[8 + 2 * i + 1] = bf_hi(vb1[i]);
    }
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      const float mn = fmaxf(m[hh], fmaxf(s0[hh], s1[hh]));
      const float f = exp2f((m[hh] - mn) * kLog2e);
      const float e0 = exp2f((s0[hh] - mn) * kLog2e);
      const float e1 = exp2f((s1[hh] - mn) * kLog2e);
      m[hh] = mn;
      l[hh] = l[hh] * f + e0 + e1;
#pragma unroll
      for (int d = 0; d < 16; ++d) o[hh][d] = fmaf(e1, vf1[d], fmaf(e0, vf0[d], o[hh][d] * f));
    }
    cur = nxt;
  }
  if (last && G == 0) {
    // the new position, from LDS
    float s0[4];
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      float x0 = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) x0 = dot2(kvnew[0][j * 8 + i], q[hh][i], x0);
      s0[hh] = tree16(x0);
    }
    float vf0[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      vf0[2 * i] = bf_lo(kvnew[1][j * 8 + i]);
      vf0[2 * i + 1] = bf_hi(kvnew[1][j * 8 + i]);
    }
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      const float mn = fmaxf(m[hh], s0[hh]);
      const float f = exp2f((m[hh] - mn) * kLog2e);
      const float e0 = exp2f((s0[hh] - mn) * kLog2e);
      m[hh] = mn;
      l[hh] = l[hh] * f + e0;
#pragma unroll
      for (int d = 0; d < 16; ++d) o[hh][d] = fmaf(e0, vf0[d], o[hh][d] * f);
    }
  }

  // ---- merge the 16 row-states of the block ----
  if (j == 0) {
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) mx[G][hh] = m[hh];
  }
  __syncthreads();
  float M[4];
#pragma unroll
  for (int hh = 0; hh < 4; ++hh) {
    float mm = mx[0][hh];
#pragma unroll
    for (int r = 1; r < 16; ++r) mm = fmaxf(mm, mx[r][hh]);
    M[hh] = mm;
    const float f = exp2f((m[hh] - mm) * kLog2e);
    l[hh] *= f;
#pragma unroll
    for (int d = 0; d < 16; ++d) o[hh][d] *= f;
  }
  // sum the four rows of the wave
#pragma unroll
  for (int hh = 0; hh < 4; ++hh) {
    l[hh] += __shfl_xor(l[hh], 16, 64);
    l[hh] += __shfl_xor(l[hh], 32, 64);
#pragma unroll
    for (int d = 0; d < 16; ++d) {
      o[hh][d] += __shfl_xor(o[hh][d], 16, 64);
      o[hh][d] += __shfl_xor(o[hh][d], 32, 64);
    }
  }
  if (grp == 0) {
#pragma unroll
    for (int hh = 0; hh < 4; ++hh)
#pragma unroll
      for (int d = 0; d < 16; ++d) osum[wave][hh][j * 16 + d] = o[hh][d];
    if (j == 0)
#pragma unroll
      for (int hh = 0; hh < 4; ++hh) lsum[wave][hh] = l[hh];
  }
  __syncthreads();
  {
    const int hh = t >> 6, d0 = (t & 63) * 4;
    const int head = 4 * g + hh;
    float4 acc;
    acc.x = osum[0][hh][d0] + osum[1][hh][d0] + osum[2][hh][d0] + osum[3][hh][d0];
    acc.y = osum[0][hh][d0 + 1] + osum[1][hh][d0 + 1] + osum[2][hh][d0 + 1] + osum[3][hh][d0 + 1];
    acc.z = osum[0][hh][d0 + 2] + osum[1][hh][d0 + 2] + osum[2][hh][d0 + 2] + osum[3][hh][d0 + 2];
    acc.w = osum[0][hh][d0 + 3] + osum[1][hh][d0 + 3] + osum[2][hh][d0 + 3] + osum[3][hh][d0 + 3];
    *reinterpret_cast<float4*>(a.part_o + ((size_t)head * S + split) * 256 + d0) = acc;
    if ((t & 63) == 0) {
      const float L = lsum[0][hh] + lsum[1][hh] + lsum[2][hh] + lsum[3][hh];
      *reinterpret_cast<float2*>(a.part_ml + ((size_t)head * S + split) * 2) = make_float2(M[hh], L);
    }
  }
}

// Grid (8 heads, 8 chunks of 32 dims). Every block recomputes the head's
// (max, sum) over the splits; thread t then sums splits t/8, t/8+32, ... for
// four dims with independent float4 loads, and 32 partial sums per dim are
// combined in a fixed order.
__global__ __launch_bounds__(256) void k_attn_merge(AttnArgs a) {
  __shared__ float scale[kMaxSplits];
  __shared__ float4 red[32][8];
  __shared__ float wred[4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int h = blockIdx.x, chunk = blockIdx.y, S = a.splits;
  const float* ml = a.part_ml + (size_t)h * S * 2;
  float mloc = -3.402823466e38f;
  for (int s = t; s < S; s += 256) mloc = fmaxf(mloc, ml[2 * s]);
  mloc = wave_max(mloc);
  if (lane == 0) wred[wave] = mloc;
  __syncthreads();
  const float M = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
  __syncthreads();
  float lloc = 0.0f;
  for (int s = t; s < S; s += 256) {
    const float f = exp2f((ml[2 * s] - M) * kLog2e);
    scale[s] = f;
    lloc += f * ml[2 * s + 1];
  }
  lloc = tree64(lloc);
  if (lane == 0) wred[wave] = lloc;
  __syncthreads();
  const float L = (wred[0] + wred[1]) + (wred[2] + wred[3]);
  const int quad = t & 7, sub = t >> 3;  // 8 quads of 4 dims, 32 split subsets
  const int d0 = chunk * 32 + quad * 4;
  const float* po = a.part_o + (size_t)h * S * 256 + d0;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
  for (int s = sub; s < S; s += 32) {
    const float4 v = *reinterpret_cast<const float4*>(po + (size_t)s * 256);
    const float f = scale[s];
    acc.x = fmaf(f, v.x, acc.x);
    acc.y = fmaf(f, v.y, acc.y);
    acc.z = fmaf(f, v.z, acc.z);
    acc.w = fmaf(f, v.w, acc.w);
  }
  red[sub][quad] = acc;
  __syncthreads();
  if (t < 32) {
    const int q = t >> 2, e = t & 3;
    float o = 0.0f;
    for (int r = 0; r < 32; ++r) {
      const float4 v = red[r][q];
      o += e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
    }
    o = L == 0.0f ? o : o / L;
    const int d = chunk * 32 + t;
    const float attention = rbf(o);
    const float gate = sigmoid_bf(bf2f(a.q_proj[h * 512 + 256 + d]));
    a.gated[h * 256 + d] = (uint16_t)f2bf(attention * gate);
  }
}

bool attn_ok(const AttnArgs& a) {
  return a.q_proj && a.k_proj && a.v_proj && a.q_gain && a.k_gain && a.kcache && a.vcache &&
         a.inv_freq && a.part_o && a.part_ml && a.gated && a.splits >= 1 &&
         a.splits <= kMaxSplits && a.capacity > 0 && (a.st || (a.pos_val >= 0 && a.pos_val < a.capacity));
}

}  // namespace

size_t attn_scratch_bytes(int splits) { return (size_t)8 * splits * (256 + 2) * sizeof(float); }

hipError_t launch_attn_split(const AttnArgs& a, hipStream_t s) {
  if (!attn_ok(a)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_split, dim3(a.splits, kKvHeads), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_attn_merge(const AttnArgs& a, hipStream_t s) {
  if (!attn_ok(a)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_merge, dim3(kQHeads, 8), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace es
