// Device-side helpers shared by the decode kernels (gfx950, wave64).
//
// bf16 values travel as raw uint16_t. f2bf is round-to-nearest-even, the
// rounding every "bfloat(x)" in the reference kernels performs. The MLX
// stepwise sigmoid and softplus keep the reference's bf16 boundaries
// (linear.metal:389-395, gdn.metal:10-29).
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
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ float bf_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

__device__ __forceinline__ uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// MLX unary sigmoid in bf16: round after exp, add, reciprocal, subtraction.
__device__ __forceinline__ float sigmoid_bf(float x) {
  float e = rbf(expf(fabsf(x)));
  float d = rbf(1.0f + e);
  float p = rbf(1.0f / d);
  return rbf(x < 0.0f ? p : 1.0f - p);
}

// MLX log1p specialised to [0,1] (utils.h), then bf16 softplus.
__device__ __forceinline__ float mlx_log1p(float x) {
  float xp1 = 1.0f + x;
  if (xp1 == 1.0f) return x;
  return x * (logf(xp1) / (xp1 - 1.0f));
}
__device__ __forceinline__ float softplus_bf(float x) {
  float e = rbf(expf(-fabsf(x)));
  float l = rbf(mlx_log1p(e));
  return rbf(fmaxf(x, 0.0f) + l);
}

// ---- wave reductions (DPP inside a 16-lane row, then cross-row shuffles) ----
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
// Sum over the 4 lanes of a quad; every lane receives the result.
__device__ __forceinline__ float quad_sum(float v) {
  v += dpp_xor1(v);
  v += dpp_xor2(v);
  return v;
}
// Sum over a 16-lane row; every lane of the row receives the result.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_xor1(v);
  v += dpp_xor2(v);
  v += dpp_half_mirror(v);
  v += dpp_mirror(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_xor1(v));
  v = fmaxf(v, dpp_xor2(v));
  v = fmaxf(v, dpp_half_mirror(v));
  v = fmaxf(v, dpp_mirror(v));
  return v;
}
// Sum over a 32-lane half wave; every lane of the half receives the result.
__device__ __forceinline__ float half_sum(float v) {
  v = row16_sum(v);
  v += __shfl_xor(v, 16, 64);
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  v = half_sum(v);
  v += __shfl_xor(v, 32, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}

// ---- Q4 affine group-64 dot over one 32-element slice ----
// codes: 4 u32 words = 32 nibbles for elements k..k+31 (nibble j of word w is
// element 8w+j, linear.metal:21). xr holds x with odd elements pre-divided by
// 16, so masking (not shifting) the odd nibbles gives exact 16*q products.
__device__ __forceinline__ float q4_dot32(const u32x4 c, const float* xr) {
  float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t word = c[w];
    uint32_t lo = word & 0x0F0F0F0Fu;
    uint32_t hi = word & 0xF0F0F0F0u;
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

// Load a 32-element bf16 slice (64 B) as floats.
__device__ __forceinline__ void load_bf16x32(const uint16_t* p, float* out) {
  const u32x4* q = reinterpret_cast<const u32x4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    u32x4 v = q[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[8 * i + 2 * j] = bf_lo(v[j]);
      out[8 * i + 2 * j + 1] = bf_hi(v[j]);
    }
  }
}

// Turn a slice of x into the register form used by q4_dot32; returns sum(x).
__device__ __forceinline__ float prep_slice(const float* x, float* xr) {
  float xs = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    xs += x[j];
    xr[j] = (j & 1) ? x[j] * 0.0625f : x[j];
  }
  return xs;
}

struct Q4 {
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  int n;
  int k;
};

// Device-resident decode cursor shared by every kernel of a step.
struct StepState {
  int pos;          // absolute position of the token consumed by this step
  int step;         // index of the output written by this step
  uint32_t token;   // token consumed by this step
  uint32_t head_counter;  // arrival counter of the vocab-head blocks
};

__device__ __forceinline__ int load_pos(const StepState* st, int pos_val) {
  return st ? st->pos : pos_val;
}

}  // namespace es
