// Device-side helpers shared by the decode kernels (gfx950, wave64).
//
// Arithmetic contract. Every kernel computes in fp32 with the bf16 rounding
// points of the reference (bf16 = round-to-nearest-even, v_cvt_pk_bf16_f32),
// and with one fixed evaluation order: fused multiply-adds only where fmaf is
// written (the library is built with -ffp-contract=off), sequential chains as
// written, and cross-lane sums as pairwise trees in lane order (tree_n below).
// exp, log and sin/cos are this file's own series evaluations, so results are
// reproducible bit for bit by a host implementation of the same steps.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace es {

constexpr int kHidden = 1024;
constexpr int kFfn = 3584;
constexpr int kGdnHeads = 16;
constexpr int kGdnDim = 128;
constexpr int kConv = 6144;       // Q|K|V conv channels, 3 x 2048
constexpr int kQHeads = 8;
constexpr int kKvHeads = 2;
constexpr int kHeadDim = 256;
constexpr int kQProj = 4096;      // 8 x (256 query + 256 gate)
constexpr int kKvProj = 512;      // 2 x 256

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));  // for the nontemporal builtins
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// ---- bf16 ----
__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ float bf_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }
__device__ __forceinline__ uint32_t f2bf(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float rbf(float f) { return (float)(__bf16)f; }
// Two values -> packed bf16 pair (lo in bits 0..15).
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// ---- series math (bit-reproducible on the host) ----
// exp: x = n ln2 + r, |r| <= ln2/2, degree-7 Taylor polynomial of e^r, scaled
// by 2^n. Inputs <= -86 give 0 (keeps every result a normal number).
__device__ __forceinline__ float es_exp(float x) {
  if (!(x > -86.0f)) return 0.0f;
  if (x > 88.72f) return __builtin_inff();
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

// log for positive normal x: x = m 2^e with m in [sqrt(1/2), sqrt(2)),
// log m = 2 atanh(s), s = (m-1)/(m+1), series to s^9.
__device__ __forceinline__ float es_log(float x) {
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

// sin and cos of an fp32 angle: quadrant reduction in double precision, then
// Taylor polynomials on |r| <= pi/4.
__device__ __forceinline__ void es_sincos(float x, float* sn, float* cs) {
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

// MLX unary sigmoid in bf16: round after exp, add, reciprocal, subtraction
// (linear.metal:389-395, gdn.metal:10-15).
__device__ __forceinline__ float sigmoid_bf(float x) {
  const float e = rbf(es_exp(fabsf(x)));
  const float d = rbf(1.0f + e);
  const float p = rbf(1.0f / d);
  return rbf(x < 0.0f ? p : 1.0f - p);
}

// MLX log1p specialised to [0,1] (utils.h, gdn.metal:19-23), bf16 softplus
// (gdn.metal:25-29).
__device__ __forceinline__ float mlx_log1p(float x) {
  const float xp1 = 1.0f + x;
  if (xp1 == 1.0f) return x;
  return x * (es_log(xp1) / (xp1 - 1.0f));
}
__device__ __forceinline__ float softplus_bf(float x) {
  const float e = rbf(es_exp(-fabsf(x)));
  const float l = rbf(mlx_log1p(e));
  return rbf(fmaxf(x, 0.0f) + l);
}

// ---- cross-lane reductions: pairwise trees in lane order ----
// DPP row ops: xor1/xor2 inside a quad, half-mirror (i <-> 7-i) and mirror
// (i <-> 15-i) inside a 16-lane row. After xor1 and xor2 every lane of a quad
// holds the quad sum, so the mirrors add whole quad/octet sums: the result is
// ((l0+l1)+(l2+l3)) + ((l4+l5)+(l6+l7)) + ... in every lane.
__device__ __forceinline__ float dpp_xor1(float v) {
  return __builtin_amdgcn_update_dpp(0.0f, v, 0xB1, 0xf, 0xf, false);
}
__device__ __forceinline__ float dpp_xor2(float v) {
  return __builtin_amdgcn_update_dpp(0.0f, v, 0x4E, 0xf, 0xf, false);
}
__device__ __forceinline__ float dpp_half_mirror(float v) {
  return __builtin_amdgcn_update_dpp(0.0f, v, 0x141, 0xf, 0xf, false);
}
__device__ __forceinline__ float dpp_mirror(float v) {
  return __builtin_amdgcn_update_dpp(0.0f, v, 0x140, 0xf, 0xf, false);
}
// Exchanges between 16-lane rows by the gfx950 row-swap instructions
// (v_permlane16_swap_b32, v_permlane32_swap_b32: VALU operations, where a
// shuffle goes through the LDS crossbar). Swapping a value with a copy of
// itself leaves in every lane the row-ordered pair (v[l & ~16], v[l | 16])
// (resp. (v[l & ~32], v[l | 32])); its sum or max equals v + v[l ^ 16]
// (v + v[l ^ 32]) bit for bit, since addition and max are commutative.
// Callers run them with the whole wave active.
__device__ __forceinline__ float2 rows_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float2 rows_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float tree4(float v) {
  v = v + dpp_xor1(v);
  v = v + dpp_xor2(v);
  return v;
}
// Sum of each group of 8 lanes, (quad 0) + (quad 1), in all its lanes.
__device__ __forceinline__ float tree8(float v) {
  v = tree4(v);
  return v + dpp_half_mirror(v);
}
__device__ __forceinline__ float tree16(float v) {
  v = tree4(v);
  v = v + dpp_half_mirror(v);
  v = v + dpp_mirror(v);
  return v;
}
__device__ __forceinline__ float tree32(float v) {
  v = tree16(v);
  const float2 p = rows_xor16(v);
  return p.x + p.y;
}
__device__ __forceinline__ float tree64(float v) {
  v = tree32(v);
  const float2 p = rows_xor32(v);
  return p.x + p.y;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_xor1(v));
  v = fmaxf(v, dpp_xor2(v));
  v = fmaxf(v, dpp_half_mirror(v));
  v = fmaxf(v, dpp_mirror(v));
  return v;
}
// Each lane keeps its own value as the first operand of the max (as with a
// shuffle), so a +0/-0 tie resolves exactly as it did lane by lane.
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  const int lane = threadIdx.x & 63;
  float2 p = rows_xor16(v);
  v = (lane & 16) ? fmaxf(p.y, p.x) : fmaxf(p.x, p.y);
  p = rows_xor32(v);
  v = (lane & 32) ? fmaxf(p.y, p.x) : fmaxf(p.x, p.y);
  return v;
}

// ---- Q4 affine group-64 dot over one 32-element slice ----
// codes: 4 u32 words = 32 nibbles for elements k..k+31 (nibble j of word w is
// element 8w+j, linear.metal:21). Two fma chains: a0 over the even elements
// in order, a1 over the odd ones; dot = a0 + a1. xr holds x with the odd
// elements pre-divided by 16, so masking (not shifting) the odd nibbles gives
// (x/16)*(16q), the same exact product as x*q.
__device__ __forceinline__ float q4_dot32(const u32x4 c, const float* xr) {
  float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t word = c[w];
    uint32_t lo = word & 0x0F0F0F0Fu;
    uint32_t hi = word & 0xF0F0F0F0u;
    // Opaque to known-bits analysis, so each byte converts with one
    // v_cvt_f32_ubyteN instead of a separate nibble extract per element.
    asm("" : "+v"(lo));
    asm("" : "+v"(hi));
    a0 = fmaf(xr[8 * w + 0], (float)(lo & 0xffu), a0);
    a1 = fmaf(xr[8 * w + 1], (float)(hi & 0xffu), a1);
    a0 = fmaf(xr[8 * w + 2], (float)((lo >> 8) & 0xffu), a0);
    a1 = fmaf(xr[8 * w + 3], (float)((hi >> 8) & 0xffu), a1);
    a0 = fmaf(xr[8 * w + 4], (float)((lo >> 16) & 0xffu), a0);
    a1 = fmaf(xr[8 * w + 5], (float)((hi >> 16) & 0xffu), a1);
    a0 = fmaf(xr[8 * w + 6], (float)(lo >> 24), a0);
    a1 = fmaf(xr[8 * w + 7], (float)(hi >> 24), a1);
  }
  return a0 + a1;
}

// Slice partial of a row: fma(xs, bias, scale * dot).
__device__ __forceinline__ float q4_slice(const u32x4 c, uint32_t scale, uint32_t bias,
                                          const float* xr, float xs) {
  return fmaf(xs, bf2f(bias), bf2f(scale) * q4_dot32(c, xr));
}

// The same with the group's scale and bias packed in one word (scale in the
// low half, bias in the high half): one load where q4_slice takes two.
__device__ __forceinline__ float q4_slice_sb(const u32x4 c, uint32_t sb, const float* xr, float xs) {
  return fmaf(xs, bf_hi(sb), bf_lo(sb) * q4_dot32(c, xr));
}

// Load a 32-element bf16 slice (64 B) as floats.
__device__ __forceinline__ void load_bf16x32(const uint16_t* p, float* out) {
  const u32x4* q = reinterpret_cast<const u32x4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 v = q[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[8 * i + 2 * j] = bf_lo(v[j]);
      out[8 * i + 2 * j + 1] = bf_hi(v[j]);
    }
  }
}

// Raw 64-byte slice (32 bf16) as four 16-byte words, for loads issued early.
struct Raw64 {
  u32x4 q[4];
};

__device__ __forceinline__ Raw64 load_raw64(const uint16_t* p) {
  const u32x4* q = reinterpret_cast<const u32x4*>(p);
  return Raw64{{q[0], q[1], q[2], q[3]}};
}

__device__ __forceinline__ void unpack_bf16x32(const Raw64& r, float* out) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[8 * i + 2 * j] = bf_lo(r.q[i][j]);
      out[8 * i + 2 * j + 1] = bf_hi(r.q[i][j]);
    }
}

// Cache-policy operand of the global->LDS and buffer load builtins that sets
// the non-temporal (streaming) hint on gfx950.
constexpr int kLoadNonTemporal = 2;

// Keeps the machine scheduler from moving instructions across this point, so
// loads issued above it are in flight before the arithmetic below starts.
__device__ __forceinline__ void issue_fence() { __builtin_amdgcn_sched_barrier(0); }

// Register form of a slice for q4_dot32; returns the sequential sum of x.
__device__ __forceinline__ float prep_slice(const float* x, float* xr) {
  float xs = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    xs = xs + x[j];
    xr[j] = (j & 1) ? x[j] * 0.0625f : x[j];
  }
  return xs;
}

// Sequential fma chain of squares over a 32-element slice.
__device__ __forceinline__ float sumsq32(const float* x) {
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) ss = fmaf(x[j], x[j], ss);
  return ss;
}

// RMSNorm of a K=1024 vector (rms_norm_bf16 arithmetic, linear.metal:311-329:
// fp32 sum of squares, bf16(bf16(x*inv)*gain)) computed once per 256-thread
// block. Every lane holds a 32-element slice (lane & 31) in xv and forms the
// inverse RMS from it: a sequential fma chain of squares over the slice, then
// tree32 over the 32 slices. Thread t normalises elements 4t..4t+3 (x4, g4:
// their bf16 values) into LDS, and after the barrier each lane reads back its
// slice. Slice k sits at lds[36k ..] so that the 16-byte reads of a half-wave
// spread over the banks.
constexpr int kNormLds = 32 * 36;
__device__ __forceinline__ void norm_block_1024(const float* xv, uint2 x4, uint2 g4, float* lds,
                                                float* xn) {
  const float ss = tree32(sumsq32(xv));
  const float inv = 1.0f / sqrtf(ss / 1024.0f + 1e-6f);
  const int t = threadIdx.x;
  const float xe[4] = {bf_lo(x4.x), bf_hi(x4.x), bf_lo(x4.y), bf_hi(x4.y)};
  const float ge[4] = {bf_lo(g4.x), bf_hi(g4.x), bf_lo(g4.y), bf_hi(g4.y)};
  float4 o;
  o.x = rbf(rbf(xe[0] * inv) * ge[0]);
  o.y = rbf(rbf(xe[1] * inv) * ge[1]);
  o.z = rbf(rbf(xe[2] * inv) * ge[2]);
  o.w = rbf(rbf(xe[3] * inv) * ge[3]);
  *reinterpret_cast<float4*>(lds + (t >> 3) * 36 + (t & 7) * 4) = o;
  __syncthreads();
  const int sl = threadIdx.x & 31;
  const float4* r = reinterpret_cast<const float4*>(lds + sl * 36);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 v = r[i];
    xn[4 * i] = v.x; xn[4 * i + 1] = v.y; xn[4 * i + 2] = v.z; xn[4 * i + 3] = v.w;
  }
}

struct Q4 {
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  int n;
  int k;
};

// Dequantised embedding slice (embedding_q4, linear.metal:20-23) of a K=1024
// table: the lane's 32 elements sl*32 .. +31 of row tok. The table is taken
// by value: a reference into the kernel-argument struct made the compiler copy
// the whole struct to per-thread scratch memory.
// The same from a slice's loaded code word and raw bf16 scale and bias.
__device__ __forceinline__ void embed_convert(const u32x4 c, uint32_t scale, uint32_t bias, float* xv) {
  const float sc = bf2f(scale), bi = bf2f(bias);
#pragma unroll
  for (int w = 0; w < 4; ++w)
#pragma unroll
    for (int j = 0; j < 8; ++j) xv[8 * w + j] = rbf(fmaf(sc, (float)((c[w] >> (4 * j)) & 15u), bi));
}
__device__ __forceinline__ void embed_slice(Q4 e, uint32_t tok, int sl, float* xv) {
  if (tok >= (uint32_t)e.n) tok = 0;  // ids come from validated prompts or the head's argmax
  const u32x4 c = *reinterpret_cast<const u32x4*>(e.w + (size_t)tok * 128 + sl * 4);
  embed_convert(c, e.s[(size_t)tok * 16 + sl / 2], e.b[(size_t)tok * 16 + sl / 2], xv);
}

// Device-resident decode cursor shared by every kernel of a step.
struct StepState {
  int pos;          // absolute position of the token consumed by this step
  int step;         // index of the output written by this step
  uint32_t token;   // token consumed by this step
  uint32_t pad;
};

__device__ __forceinline__ int load_pos(const StepState* st, int pos_val) {
  return st ? st->pos : pos_val;
}



__device__ __forceinline__ void store_bf16x32(uint16_t* p, const float* v) {
  u32x4* q = reinterpret_cast<u32x4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = pack_bf2(v[8 * i + 2 * j], v[8 * i + 2 * j + 1]);
    q[i] = o;
  }
}

// ---- shared by the decode and the row-batched (prefill) kernels ----

// Causal conv1d of one channel over taps (oldest first) + SiLU with the MLX
// bf16 steps (gdn_input.metal:163-170): x = bf16(fma chain), bf16(x*sigmoid_bf(x)).
__device__ __forceinline__ float conv4_silu(const uint32_t* x, uint2 w) {
  float acc = 0.0f;
  acc = fmaf(bf2f(x[0]), bf_lo(w.x), acc);
  acc = fmaf(bf2f(x[1]), bf_hi(w.x), acc);
  acc = fmaf(bf2f(x[2]), bf_lo(w.y), acc);
  acc = fmaf(bf2f(x[3]), bf_hi(w.y), acc);
  const float xv = rbf(acc);
  return rbf(xv * sigmoid_bf(xv));
}

// RMSNorm of a 1024-wide row held as 32-element slices by the 32 lanes of a
// half-wave (rms_norm_bf16 rounding points, linear.metal:311-329): sum of
// squares by slice (fma chain) then tree32, out = bf16(bf16(x*inv)*gain).
__device__ __forceinline__ void norm_slice_1024(const float* xv, const Raw64& gain, float* xn) {
  const float ss = tree32(sumsq32(xv));
  const float inv = 1.0f / sqrtf(ss / 1024.0f + 1e-6f);
  float gv[32];
  unpack_bf16x32(gain, gv);
#pragma unroll
  for (int j = 0; j < 32; ++j) xn[j] = rbf(rbf(xv[j] * inv) * gv[j]);
}

// Normalise 4 consecutive dims of a 256-wide head held by a full wave.
// xv, gv: the lane's 4 bf16 values of the head and of the gain.
__device__ __forceinline__ void head_norm4(const uint2 xv, const uint2 gv, float* out) {
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
// d < 32: fma(lo, c, -(hi*s)); 32 <= d < 64: fma(lo, s, hi*c), where lo and
// hi are dims d & 31 and (d & 31) + 32. own is dim d, partner dim d ^ 32;
// inv is inv_freq[d & 31] (only used for d < 64).
__device__ __forceinline__ float rope_at(float own, float partner, int d, int pos, float inv) {
  if (d >= 64) return own;
  const float angle = (float)pos * inv;
  float s, c;
  es_sincos(angle, &s, &c);
  const float lo = d < 32 ? own : partner, hi = d < 32 ? partner : own;
  return rbf(d < 32 ? fmaf(lo, c, -(hi * s)) : fmaf(lo, s, hi * c));
}

// Value of lane l ^ 8 inside each 16-lane row (DPP row rotate by 8). With 4
// dims per lane, dim d ^ 32 of a head (d < 64) sits in lane ^ 8.
__device__ __forceinline__ float dpp_row_ror8(float v) {
  return __builtin_amdgcn_update_dpp(0.0f, v, 0x128, 0xf, 0xf, false);
}

}  // namespace es
