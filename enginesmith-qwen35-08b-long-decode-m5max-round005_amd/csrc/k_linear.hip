// Q4 affine (group 64) dequant-matvec kernels for batch-1 decode on gfx950.
//
// Layout is the reference's (weights.rs:50-52): codes u32 [N, K/8] with 8
// nibbles per word (nibble j of word w = column 8w+j), bf16 scale and bias per
// 64 columns. A lane owns one 32-column slice of a row (one 16-byte code load,
// half a group); a K=1024 row is one half-wave, wider rows loop over slices.
// Each lane keeps its slice of x in registers, so the only per-row traffic is
// the 16-byte code load plus one scale and one bias. Accumulation is fp32 and
// the result is rounded to bf16 once (linear.metal:41-72); the residual
// epilogue rounds the projection before the add (linear.metal:121).
//
// Evaluation order (fixed, see es_device.hpp): slice partial
// fma(xs, bias, scale * (even-fma-chain + odd-fma-chain)); K=1024 rows sum
// their 32 slices with tree32, K=2048 rows their 64 slices with tree64, and a
// K=3584 lane l first adds slice l+64 (l < 48) to slice l, then tree64.
// Weight loads are issued at kernel entry, before the input and its RMSNorm,
// so their latency overlaps that work.
#include "es_kernels.hpp"

namespace es {
namespace {

struct MultiDev {
  Q4 m[4];
  uint16_t* y[4];
  int count;
  int total;
  int ring0;
  const uint16_t* x;
  const float* dpart;
  const uint16_t* gain;
  uint16_t* norm_out;
  Q4 embed;
  uint16_t* h_out;
  uint32_t token_val;
  const StepState* st;
  int pos_val;
};

// Input modes of k_norm_multi: the vector x; the embedding row of the step's
// token; x plus the down projection's eight octet partials (k_mlp_xcd).
constexpr int kInX = 0, kInEmbed = 1, kInParts = 2;

template <int P, int IN>
__global__ __launch_bounds__(256) void k_norm_multi(MultiDev a) {
  constexpr bool EMBED = IN == kInEmbed, PARTS = IN == kInParts;
  const int lane = threadIdx.x & 63, half = lane >> 5, sl = lane & 31;
  // A wave's 2P rows lie in one matrix (every matrix has a multiple of 2P
  // rows), so the matrix and its pointers are wave-uniform (scalar registers).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wrow0 = (blockIdx.x * 4 + wave) * (2 * P);
  const bool wvalid = wrow0 < a.total;
  int m = 0, local0 = wvalid ? wrow0 : 0;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    if (m == i && i + 1 < a.count && local0 >= a.m[i].n) {
      local0 -= a.m[i].n;
      m = i + 1;
    }
  }
  const Q4 q = m == 0 ? a.m[0] : m == 1 ? a.m[1] : m == 2 ? a.m[2] : a.m[3];
  // Input, gain and position loads first, then the weights. Loads complete
  // in issue order, so the normalisation (which needs only the input) runs
  // while the weights are still arriving; issued the other way round it
  // would wait for every weight load. The weights are non-temporal: the
  // input projections (94 MB per step) are left out of the on-package cache
  // so that the other layer weights (about 200 MB) stay in it from one step
  // to the next.
  __shared__ float norm_lds[kNormLds];
  __shared__ float hs[PARTS ? kNormLds : 1];
  const Raw64 graw = EMBED ? load_raw64(a.gain + sl * 32) : Raw64{};
  uint2 x4 = EMBED ? uint2{0u, 0u} : reinterpret_cast<const uint2*>(a.x)[threadIdx.x];
  const uint2 g4 = EMBED ? uint2{0u, 0u} : reinterpret_cast<const uint2*>(a.gain)[threadIdx.x];
  float4 dp[PARTS ? 8 : 1];
  if (PARTS) {
#pragma unroll
    for (int k = 0; k < 8; ++k) dp[k] = reinterpret_cast<const float4*>(a.dpart + k * kHidden)[threadIdx.x];
  }
  // Ring slot of the first output: the step's position (read early, used at the store).
  int zero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
  const int* pos_src = a.st ? &a.st->pos : reinterpret_cast<const int*>(a.gain);
  const int pos_raw = pos_src[zero];
  const Raw64 xraw = EMBED || PARTS ? Raw64{} : load_raw64(a.x + sl * 32);
  issue_fence();
  u32x4 c[P];
  uint32_t sv[P], bv[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int local = local0 + 2 * p + half;
    c[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(q.w + (size_t)local * 128 + sl * 4));
    sv[p] = __builtin_nontemporal_load(q.s + (size_t)local * 16 + sl / 2);
    bv[p] = __builtin_nontemporal_load(q.b + (size_t)local * 16 + sl / 2);
  }
  issue_fence();
  float xv[32];
  if (EMBED) {
    const uint32_t tok = a.st ? a.st->token : a.token_val;
    embed_slice(a.embed, tok, sl, xv);
    if (a.h_out && blockIdx.x == 0 && threadIdx.x < 32) store_bf16x32(a.h_out + sl * 32, xv);
  } else if (PARTS) {
    // x = bf16(x + bf16(pairwise sum of the eight octet partials)), the down
    // projection's residual epilogue; thread t forms elements 4t..4t+3 and
    // they pass through LDS so every lane also has its 32-element slice
    const int t = threadIdx.x;
    const float hf[4] = {bf_lo(x4.x), bf_hi(x4.x), bf_lo(x4.y), bf_hi(x4.y)};
    float hn[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float c[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) c[k] = e == 0 ? dp[k].x : e == 1 ? dp[k].y : e == 2 ? dp[k].z : dp[k].w;
      hn[e] = bf2f(f2bf(hf[e] + rbf(((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7])))));
    }
    x4 = make_uint2(pack_bf2(hn[0], hn[1]), pack_bf2(hn[2], hn[3]));
    if (a.h_out && blockIdx.x == 0) reinterpret_cast<uint2*>(a.h_out)[t] = x4;
    *reinterpret_cast<float4*>(hs + (t >> 3) * 36 + (t & 7) * 4) = make_float4(hn[0], hn[1], hn[2], hn[3]);
    __syncthreads();
    const float4* rp = reinterpret_cast<const float4*>(hs + sl * 36);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 q = rp[i];
      xv[4 * i] = q.x; xv[4 * i + 1] = q.y; xv[4 * i + 2] = q.z; xv[4 * i + 3] = q.w;
    }
  } else {
    unpack_bf16x32(xraw, xv);
  }
  float xn[32];
  if (EMBED) norm_slice_1024(xv, graw, xn);
  else norm_block_1024(xv, x4, g4, norm_lds, xn);
  if (a.norm_out && blockIdx.x == 0 && threadIdx.x < 32) store_bf16x32(a.norm_out + sl * 32, xn);
  float xr[32];
  const float xs = prep_slice(xn, xr);

  uint16_t* y = m == 0 ? a.y[0] : m == 1 ? a.y[1] : m == 2 ? a.y[2] : a.y[3];
  if (m == 0 && a.ring0) y += (size_t)((a.st ? pos_raw : a.pos_val) & 3) * a.m[0].n;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const float part = tree32(q4_slice(c[p], sv[p], bv[p], xr, xs));
    if (sl == 0 && wvalid) y[local0 + 2 * p + half] = (uint16_t)f2bf(part);
  }
}

// RMSNorm + gate/up projections + SwiGLU with the MLX bf16 graph boundaries
// (linear_norm.metal:88-102). A wave owns 2*NP output rows; lane 0 of each
// half holds a row's gate and up sums and applies the activation in place.
template <int NP>
__global__ __launch_bounds__(256) void k_norm_gate_up(Q4 gate, Q4 up, const uint16_t* x,
                                                      const uint16_t* gain, uint16_t* norm_out,
                                                      uint16_t* act) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5, sl = lane & 31;
  const int base = (blockIdx.x * 4 + wave) * (2 * NP);
  // Input and gain first, then the weights (loads complete in issue order:
  // the normalisation runs while the weights arrive).
  __shared__ float norm_lds[kNormLds];
  const Raw64 xraw = load_raw64(x + sl * 32);
  const uint2 x4 = reinterpret_cast<const uint2*>(x)[threadIdx.x];
  const uint2 g4 = reinterpret_cast<const uint2*>(gain)[threadIdx.x];
  issue_fence();
  u32x4 cg[NP], cu[NP];
  uint32_t sg[NP], bg[NP], su[NP], bu[NP];
  int rr[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int r = base + 2 * p + half;
    rr[p] = r;
    const int rl = r < gate.n ? r : 0;
    cg[p] = *reinterpret_cast<const u32x4*>(gate.w + (size_t)rl * 128 + sl * 4);
    cu[p] = *reinterpret_cast<const u32x4*>(up.w + (size_t)rl * 128 + sl * 4);
    sg[p] = gate.s[(size_t)rl * 16 + sl / 2];
    bg[p] = gate.b[(size_t)rl * 16 + sl / 2];
    su[p] = up.s[(size_t)rl * 16 + sl / 2];
    bu[p] = up.b[(size_t)rl * 16 + sl / 2];
  }
  issue_fence();
  float xv[32];
  unpack_bf16x32(xraw, xv);
  float xn[32];
  norm_block_1024(xv, x4, g4, norm_lds, xn);
  if (norm_out && blockIdx.x == 0 && threadIdx.x < 32) store_bf16x32(norm_out + sl * 32, xn);
  float xr[32];
  const float xs = prep_slice(xn, xr);
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const float g = tree32(q4_slice(cg[p], sg[p], bg[p], xr, xs));
    const float u = tree32(q4_slice(cu[p], su[p], bu[p], xr, xs));
    if (sl == 0 && rr[p] < gate.n) {
      const float gb = rbf(g), ub = rbf(u);
      const float silu = rbf(gb * sigmoid_bf(gb));
      act[rr[p]] = (uint16_t)f2bf(silu * ub);
    }
  }
}

// Pairwise sum of N head partials in index order (the upper levels of the
// 64-slice row tree).
template <int N>
__device__ __forceinline__ float pair_sum(const float* v) {
  if constexpr (N == 1) {
    return v[0];
  } else {
    return pair_sum<N / 2>(v) + pair_sum<N / 2>(v + N / 2);
  }
}

// As k_norm_gate_up, but the input is formed here from the previous
// projection's head partials: h = bf16(h_old + bf16(pair_sum(partials)))
// (the residual epilogue of the K=2048 projection), written to h_new by block
// 0 for the next launch's residual. Thread t forms elements 4t..4t+3; they
// pass through LDS so every lane also has its 32-element slice.
template <int NP, int NPART>
__global__ __launch_bounds__(256) void k_norm_gate_up_parts(Q4 gate, Q4 up, const uint16_t* h_old,
                                                            const float* part, uint16_t* h_new,
                                                            const uint16_t* gain, uint16_t* act) {
  __shared__ float hs[kNormLds];
  __shared__ float norm_lds[kNormLds];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6, half = lane >> 5, sl = lane & 31;
  const int base = (blockIdx.x * 4 + wave) * (2 * NP);
  // The residual, gain and partials first, then the weights (loads complete
  // in issue order: the partial sum and the normalisation run while the
  // weights arrive).
  const uint2 ho = reinterpret_cast<const uint2*>(h_old)[t];
  const uint2 g4 = reinterpret_cast<const uint2*>(gain)[t];
  float4 pv[NPART];
#pragma unroll
  for (int k = 0; k < NPART; ++k) pv[k] = reinterpret_cast<const float4*>(part + k * kHidden)[t];
  issue_fence();
  u32x4 cg[NP], cu[NP];
  uint32_t sg[NP], bg[NP], su[NP], bu[NP];
  int rr[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int r = base + 2 * p + half;
    rr[p] = r;
    const int rl = r < gate.n ? r : 0;
    cg[p] = *reinterpret_cast<const u32x4*>(gate.w + (size_t)rl * 128 + sl * 4);
    cu[p] = *reinterpret_cast<const u32x4*>(up.w + (size_t)rl * 128 + sl * 4);
    sg[p] = gate.s[(size_t)rl * 16 + sl / 2];
    bg[p] = gate.b[(size_t)rl * 16 + sl / 2];
    su[p] = up.s[(size_t)rl * 16 + sl / 2];
    bu[p] = up.b[(size_t)rl * 16 + sl / 2];
  }
  issue_fence();
  float hn[4];
  {
    const float hf[4] = {bf_lo(ho.x), bf_hi(ho.x), bf_lo(ho.y), bf_hi(ho.y)};
    float c[NPART];
#pragma unroll
    for (int k = 0; k < NPART; ++k) c[k] = pv[k].x;
    hn[0] = bf2f(f2bf(hf[0] + rbf(pair_sum<NPART>(c))));
#pragma unroll
    for (int k = 0; k < NPART; ++k) c[k] = pv[k].y;
    hn[1] = bf2f(f2bf(hf[1] + rbf(pair_sum<NPART>(c))));
#pragma unroll
    for (int k = 0; k < NPART; ++k) c[k] = pv[k].z;
    hn[2] = bf2f(f2bf(hf[2] + rbf(pair_sum<NPART>(c))));
#pragma unroll
    for (int k = 0; k < NPART; ++k) c[k] = pv[k].w;
    hn[3] = bf2f(f2bf(hf[3] + rbf(pair_sum<NPART>(c))));
  }
  const uint2 x4 = make_uint2(pack_bf2(hn[0], hn[1]), pack_bf2(hn[2], hn[3]));
  if (blockIdx.x == 0) reinterpret_cast<uint2*>(h_new)[t] = x4;
  *reinterpret_cast<float4*>(hs + (t >> 3) * 36 + (t & 7) * 4) = make_float4(hn[0], hn[1], hn[2], hn[3]);
  __syncthreads();
  float xv[32];
  {
    const float4* r = reinterpret_cast<const float4*>(hs + sl * 36);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 q = r[i];
      xv[4 * i] = q.x; xv[4 * i + 1] = q.y; xv[4 * i + 2] = q.z; xv[4 * i + 3] = q.w;
    }
  }
  float xn[32];
  norm_block_1024(xv, x4, g4, norm_lds, xn);
  float xr[32];
  const float xs = prep_slice(xn, xr);
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const float g = tree32(q4_slice(cg[p], sg[p], bg[p], xr, xs));
    const float u = tree32(q4_slice(cu[p], su[p], bu[p], xr, xs));
    if (sl == 0 && rr[p] < gate.n) {
      const float gb = rbf(g), ub = rbf(u);
      const float silu = rbf(gb * sigmoid_bf(gb));
      act[rr[p]] = (uint16_t)f2bf(silu * ub);
    }
  }
}

// Plain / residual QMV for K == 1024 (half-wave rows).
// Token rows (qmv_q4 with M rows, linear.metal:28-73) are grid.y: row t reads
// x[t] and residual[t] and writes y[t]; every row has the M = 1 arithmetic.
template <int P, bool ADD>
__global__ __launch_bounds__(256) void k_qmv_narrow(Q4 m, const uint16_t* x,
                                                    const uint16_t* residual, uint16_t* y,
                                                    float* y_f32) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5, sl = lane & 31;
  x += (size_t)blockIdx.y * m.k;
  y += (size_t)blockIdx.y * m.n;
  if (ADD) residual += (size_t)blockIdx.y * m.n;
  const int base = (blockIdx.x * 4 + wave) * (2 * P);
  u32x4 c[P];
  uint32_t sv[P], bv[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int r = base + 2 * p + half;
    const int rl = r < m.n ? r : 0;
    c[p] = *reinterpret_cast<const u32x4*>(m.w + (size_t)rl * 128 + sl * 4);
    sv[p] = m.s[(size_t)rl * 16 + sl / 2];
    bv[p] = m.b[(size_t)rl * 16 + sl / 2];
  }
  uint32_t res[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int r = base + 2 * p + half;
    res[p] = ADD ? residual[r < m.n ? r : 0] : 0u;
  }
  const Raw64 xraw = load_raw64(x + sl * 32);
  issue_fence();
  float xv[32], xr[32];
  unpack_bf16x32(xraw, xv);
  const float xs = prep_slice(xv, xr);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int r = base + 2 * p + half;
    const float part = tree32(q4_slice(c[p], sv[p], bv[p], xr, xs));
    if (sl == 0 && r < m.n) {
      if (y_f32) y_f32[r] = part;
      if (ADD) y[r] = (uint16_t)f2bf(bf2f(res[p]) + rbf(part));
      else y[r] = (uint16_t)f2bf(part);
    }
  }
}

// Wide rows (1024 < K <= 4096): a whole wave per row, lane slices l and l+64.
template <int P, bool ADD>
__global__ __launch_bounds__(256) void k_qmv_wide(Q4 m, const uint16_t* x,
                                                  const uint16_t* residual, uint16_t* y,
                                                  float* y_f32) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  x += (size_t)blockIdx.y * m.k;  // token row (see k_qmv_narrow)
  y += (size_t)blockIdx.y * m.n;
  if (ADD) residual += (size_t)blockIdx.y * m.n;
  const int ns = m.k >> 5;
  const bool v1 = lane < ns, v2 = lane + 64 < ns;
  const int wpr = m.k >> 3, gpr = m.k >> 6;
  const int s1 = v1 ? lane : 0, s2 = v2 ? lane + 64 : 0;
  const int base = (blockIdx.x * 4 + wave) * P;
  // Input first, then the weights (loads complete in issue order: the
  // input's slice sums and scaling run while the weights arrive).
  const Raw64 xa = load_raw64(x + s1 * 32);
  const Raw64 xb = load_raw64(x + s2 * 32);
  issue_fence();
  u32x4 c1[P], c2[P];
  uint32_t sa[P], ba[P], sb[P], bb[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int r = base + p;
    const size_t rl = r < m.n ? r : 0;
    // Slices past the row end (lanes >= K/32) load slice 0 and are masked below.
    c1[p] = *reinterpret_cast<const u32x4*>(m.w + rl * wpr + s1 * 4);
    sa[p] = m.s[rl * gpr + s1 / 2];
    ba[p] = m.b[rl * gpr + s1 / 2];
    c2[p] = *reinterpret_cast<const u32x4*>(m.w + rl * wpr + s2 * 4);
    sb[p] = m.s[rl * gpr + s2 / 2];
    bb[p] = m.b[rl * gpr + s2 / 2];
  }
  uint32_t res[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int r = base + p;
    res[p] = ADD ? residual[r < m.n ? r : 0] : 0u;
  }
  issue_fence();
  float xv[32], xr1[32], xr2[32];
  float xs1 = 0.0f, xs2 = 0.0f;
  if (v1) {
    unpack_bf16x32(xa, xv);
    xs1 = prep_slice(xv, xr1);
  } else {
#pragma unroll
    for (int j = 0; j < 32; ++j) xr1[j] = 0.0f;
  }
  if (v2) {
    unpack_bf16x32(xb, xv);
    xs2 = prep_slice(xv, xr2);
  } else {
#pragma unroll
    for (int j = 0; j < 32; ++j) xr2[j] = 0.0f;
  }
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int r = base + p;
    const float p1 = q4_slice(c1[p], sa[p], ba[p], xr1, xs1);
    const float p2 = q4_slice(c2[p], sb[p], bb[p], xr2, xs2);
    float part = v1 ? p1 : 0.0f;
    if (v2) part = part + p2;
    part = tree64(part);
    if (lane == 0 && r < m.n) {
      if (y_f32) y_f32[r] = part;
      if (ADD) y[r] = (uint16_t)f2bf(bf2f(res[p]) + rbf(part));
      else y[r] = (uint16_t)f2bf(part);
    }
  }
}

// Gated RMSNorm (gdn.metal:238-254) computed once per block into LDS, then
// out_proj (K=2048) with residual. Element k lives at xg[k + k/32] so each
// lane's 32-element slice reads without bank conflicts.
template <int P>
__global__ __launch_bounds__(256) void k_gdn_gate_out(Q4 m, const uint16_t* y, const uint16_t* z,
                                                      const uint16_t* norm_w, uint16_t* h,
                                                      uint16_t* gated_out) {
  __shared__ float xg[2048 + 64];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int base = (blockIdx.x * 4 + wave) * P;
  u32x4 c[P];
  uint32_t sv[P], bv[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int r = base + p;
    const size_t rl = r < m.n ? r : 0;
    c[p] = *reinterpret_cast<const u32x4*>(m.w + rl * 256 + lane * 4);
    sv[p] = m.s[rl * 32 + lane / 2];
    bv[p] = m.b[rl * 32 + lane / 2];
  }
  uint32_t res[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int r = base + p;
    res[p] = h[r < m.n ? r : 0];
  }
  {
    const int e0 = (t >> 4) * 128 + (t & 15) * 8;  // head t/16, eight channels
    const u32x4 yv = *reinterpret_cast<const u32x4*>(y + e0);
    const u32x4 zv = *reinterpret_cast<const u32x4*>(z + e0);
    const u32x4 wv = *reinterpret_cast<const u32x4*>(norm_w + (t & 15) * 8);
    issue_fence();
    float yf[8], zf[8], wf[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      yf[2 * j] = bf_lo(yv[j]); yf[2 * j + 1] = bf_hi(yv[j]);
      zf[2 * j] = bf_lo(zv[j]); zf[2 * j + 1] = bf_hi(zv[j]);
      wf[2 * j] = bf_lo(wv[j]); wf[2 * j + 1] = bf_hi(wv[j]);
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(yf[i], yf[i], ss);
    ss = tree16(ss);
    const float inv = 1.0f / sqrtf(ss / 128.0f + 1e-6f);
    uint32_t packed[4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float norm = rbf(rbf(yf[i] * inv) * wf[i]);
      const float gz = zf[i];
      const float sy = 1.0f / (1.0f + es_exp(fabsf(gz)));
      const float sig = gz < 0.0f ? sy : 1.0f - sy;
      const float g = rbf((gz * sig) * norm);
      const int e = e0 + i;
      xg[e + (e >> 5)] = g;
      if (i & 1) packed[i >> 1] |= f2bf(g) << 16;
      else packed[i >> 1] = f2bf(g);  // f2bf zero-extends
    }
    if (gated_out && blockIdx.x == 0)
      *reinterpret_cast<u32x4*>(gated_out + e0) = u32x4{packed[0], packed[1], packed[2], packed[3]};
  }
  __syncthreads();
  float xv[32], xr[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) xv[j] = xg[lane * 33 + j];
  const float xs = prep_slice(xv, xr);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int r = base + p;
    const float part = tree64(q4_slice(c[p], sv[p], bv[p], xr, xs));
    if (lane == 0 && r < m.n) h[r] = (uint16_t)f2bf(bf2f(res[p]) + rbf(part));
  }
}

__global__ __launch_bounds__(256) void k_embedding(Q4 e, const uint32_t* token, uint16_t* out) {
  uint32_t tok = *token;
  if (tok >= (uint32_t)e.n) tok = 0;
  for (int k = threadIdx.x; k < e.k; k += blockDim.x) {
    const uint32_t q = (e.w[(size_t)tok * (e.k / 8) + k / 8] >> (4 * (k % 8))) & 15u;
    const size_t g = (size_t)tok * (e.k / 64) + k / 64;
    out[k] = (uint16_t)f2bf(fmaf(bf2f(e.s[g]), (float)q, bf2f(e.b[g])));
  }
}

__global__ __launch_bounds__(256) void k_add_bf16(const uint16_t* a, const uint16_t* b, int count,
                                                  uint16_t* out) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < count) out[i] = (uint16_t)f2bf(bf2f(a[i]) + bf2f(b[i]));
}

bool q4_ok(const Q4& m) { return m.w && m.s && m.b && m.n > 0 && m.k > 0 && m.k % 64 == 0; }

}  // namespace

constexpr int kMultiP = 4;     // passes per wave: 8 rows per wave, 32 per block
constexpr int kGateUpNP = 2;   // 4 output rows per wave, 16 per block
constexpr int kNarrowP = 2;    // 4 rows per wave
constexpr int kWideP = 1;      // 1 row per wave
constexpr int kGateOutP = 2;   // 2 rows per wave, 8 per block

hipError_t launch_norm_multi(const NormMultiArgs& a, hipStream_t s) {
  if (a.count < 1 || a.count > 4 || !a.gain || (!a.x && !a.embed.w)) return hipErrorInvalidValue;
  MultiDev d{};
  int total = 0;
  for (int i = 0; i < a.count; ++i) {
    if (!q4_ok(a.m[i]) || a.m[i].k != kHidden || !a.y[i] || a.m[i].n % (2 * kMultiP) != 0)
      return hipErrorInvalidValue;
    d.m[i] = a.m[i];
    d.y[i] = a.y[i];
    total += a.m[i].n;
  }
  if (a.embed.w && a.embed.k != kHidden) return hipErrorInvalidValue;
  if (a.ring0 && !a.st) {
    if (a.pos_val < 0) return hipErrorInvalidValue;
  }
  if (a.dpart && (a.embed.w || !a.x)) return hipErrorInvalidValue;
  d.count = a.count;
  d.total = total;
  d.ring0 = a.ring0;
  d.x = a.x;
  d.dpart = a.dpart;
  d.gain = a.gain;
  d.norm_out = a.norm_out;
  d.embed = a.embed;
  d.h_out = a.h_out;
  d.token_val = a.token_val;
  d.st = a.st;
  d.pos_val = a.pos_val;
  const int rows_per_block = 4 * 2 * kMultiP;
  const int blocks = (total + rows_per_block - 1) / rows_per_block;
  if (a.embed.w)
    hipLaunchKernelGGL((k_norm_multi<kMultiP, kInEmbed>), dim3(blocks), dim3(256), 0, s, d);
  else if (a.dpart)
    hipLaunchKernelGGL((k_norm_multi<kMultiP, kInParts>), dim3(blocks), dim3(256), 0, s, d);
  else
    hipLaunchKernelGGL((k_norm_multi<kMultiP, kInX>), dim3(blocks), dim3(256), 0, s, d);
  return hipGetLastError();
}

hipError_t launch_norm_gate_up(const Q4& gate, const Q4& up, const uint16_t* x,
                               const uint16_t* gain, uint16_t* norm_out, uint16_t* act,
                               hipStream_t s) {
  if (!q4_ok(gate) || !q4_ok(up) || gate.k != kHidden || up.k != kHidden || gate.n != up.n ||
      !x || !gain || !act)
    return hipErrorInvalidValue;
  const int rows_per_block = 4 * 2 * kGateUpNP;
  const int blocks = (gate.n + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL(k_norm_gate_up<kGateUpNP>, dim3(blocks), dim3(256), 0, s, gate, up, x, gain,
                     norm_out, act);
  return hipGetLastError();
}

hipError_t launch_norm_gate_up_parts(const Q4& gate, const Q4& up, const uint16_t* h_old,
                                     const float* part, int nparts, uint16_t* h_new,
                                     const uint16_t* gain, uint16_t* act, hipStream_t s) {
  if (!q4_ok(gate) || !q4_ok(up) || gate.k != kHidden || up.k != kHidden || gate.n != up.n ||
      !h_old || !part || !h_new || h_new == h_old || !gain || !act)
    return hipErrorInvalidValue;
  const int rows_per_block = 4 * 2 * kGateUpNP;
  const int blocks = (gate.n + rows_per_block - 1) / rows_per_block;
  if (nparts == 16)
    hipLaunchKernelGGL((k_norm_gate_up_parts<kGateUpNP, 16>), dim3(blocks), dim3(256), 0, s, gate, up,
                       h_old, part, h_new, gain, act);
  else if (nparts == 8)
    hipLaunchKernelGGL((k_norm_gate_up_parts<kGateUpNP, 8>), dim3(blocks), dim3(256), 0, s, gate, up,
                       h_old, part, h_new, gain, act);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_qmv_rows(const Q4& w, const uint16_t* x, int rows, const uint16_t* residual,
                           uint16_t* y, float* y_f32, hipStream_t s) {
  if (!q4_ok(w) || !x || !y || rows < 1 || rows > 65535 || (y_f32 && rows != 1))
    return hipErrorInvalidValue;
  if (w.k == kHidden) {
    const int rpb = 4 * 2 * kNarrowP;
    const dim3 grid((w.n + rpb - 1) / rpb, rows);
    if (residual)
      hipLaunchKernelGGL((k_qmv_narrow<kNarrowP, true>), grid, dim3(256), 0, s, w, x, residual, y, y_f32);
    else
      hipLaunchKernelGGL((k_qmv_narrow<kNarrowP, false>), grid, dim3(256), 0, s, w, x, residual, y, y_f32);
  } else if (w.k > kHidden && w.k <= 4096) {
    const int rpb = 4 * kWideP;
    const dim3 grid((w.n + rpb - 1) / rpb, rows);
    if (residual)
      hipLaunchKernelGGL((k_qmv_wide<kWideP, true>), grid, dim3(256), 0, s, w, x, residual, y, y_f32);
    else
      hipLaunchKernelGGL((k_qmv_wide<kWideP, false>), grid, dim3(256), 0, s, w, x, residual, y, y_f32);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_qmv(const Q4& w, const uint16_t* x, const uint16_t* residual, uint16_t* y,
                      float* y_f32, hipStream_t s) {
  return launch_qmv_rows(w, x, 1, residual, y, y_f32, s);
}

int qmv_row_limit(int n, int k) {
  if (k <= 2048 && n <= 2048) return 33;
  if (k <= 4096 && n <= 4096) return 25;
  return 13;
}

hipError_t launch_gdn_gate_out(const Q4& w, const uint16_t* y, const uint16_t* z,
                               const uint16_t* norm_w, uint16_t* h, uint16_t* gated_out,
                               hipStream_t s) {
  if (!q4_ok(w) || w.k != 2048 || w.n != kHidden || !y || !z || !norm_w || !h)
    return hipErrorInvalidValue;
  const int rpb = 4 * kGateOutP;
  const int blocks = (w.n + rpb - 1) / rpb;
  hipLaunchKernelGGL(k_gdn_gate_out<kGateOutP>, dim3(blocks), dim3(256), 0, s, w, y, z, norm_w, h,
                     gated_out);
  return hipGetLastError();
}

hipError_t launch_add_bf16(const uint16_t* a, const uint16_t* b, int count, uint16_t* out, hipStream_t s) {
  if (!a || !b || !out || count < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_add_bf16, dim3((count + 255) / 256), dim3(256), 0, s, a, b, count, out);
  return hipGetLastError();
}

hipError_t launch_embedding(const Q4& table, const uint32_t* token_dev, uint16_t* out,
                            hipStream_t s) {
  if (!q4_ok(table) || !token_dev || !out) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_embedding, dim3(1), dim3(256), 0, s, table, token_dev, out);
  return hipGetLastError();
}

}  // namespace es
