// Gated DeltaNet decode step on gfx950: causal conv1d (4 taps) + SiLU, Q/K
// L2 normalisation, decay/beta gates and the delta-rule state update with
// readout, fused in one launch.
//
// Grid: 8 row-blocks x 16 heads, 256 threads. A block owns 16 value rows of
// one head; its fp32 state slice (16 x 128 = 8 KiB) is read once into
// registers, updated and written back, 16 lanes per row and 8 keys per lane
// (one DPP row per value row). Every block of a head recomputes the head's
// 256 Q/K conv channels (cheap) so no cross-block dependency exists.
//
// Convolution history is a 4-slot ring of raw projections, slot = position&3:
// the projection kernel writes slot pos&3, this kernel reads slots pos-3..pos,
// and nothing is shifted. Slots for positions < 0 are zero after reset, which
// matches the reference's zeroed [3,6144] history (gdn.metal:141-153).
//
// Arithmetic follows gdn.metal:121-171 (conv/prepare: fma over taps, bf16 at
// conv and SiLU, rsqrt(ss/128 + 1e-6/128), q x 1/128, k x bf16(128^-1/2),
// g = exp(-exp(A_log) * softplus_bf(bf16(a+dt))), beta = sigmoid_bf(b)) and
// gdn.metal:192-226 (decay, memory, delta, update, readout; fp32 state).
// Order: Q/K sum of squares = tree64 over channels 0..63 plus tree64 over
// 64..127; memory and readout = per-lane fma chains over 8 keys, tree16 over
// the 16 lanes of a row.
#include "es_kernels.hpp"

namespace es {
namespace {

// Raw values of channel c in all four ring slots, loaded before the position
// is known; conv_silu then orders them as taps (pos-3 .. pos).
struct RingTaps {
  uint32_t v[4];
  uint2 w;
};

__device__ __forceinline__ void ring_load(const uint16_t* ring, const uint16_t* conv_w, int c,
                                          RingTaps& r) {
#pragma unroll
  for (int s = 0; s < 4; ++s) r.v[s] = ring[(size_t)s * kConv + c];
  r.w = *reinterpret_cast<const uint2*>(conv_w + (size_t)c * 4);
}

__device__ __forceinline__ float conv_silu(const RingTaps& r, int pos) {
  const int sh = pos + 1;  // slot of tap t is (pos - 3 + t) & 3 = (pos + 1 + t) & 3
  uint32_t x[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int slot = (sh + t) & 3;
    x[t] = slot == 0 ? r.v[0] : slot == 1 ? r.v[1] : slot == 2 ? r.v[2] : r.v[3];
  }
  return conv4_silu(x, r.w);
}

__global__ __launch_bounds__(256) void k_gdn_recur(GdnRecurArgs a) {
  __shared__ float qk[256];
  __shared__ float vv[16];
  __shared__ float red[4];
  __shared__ float gates[2];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int h = blockIdx.y, r0 = blockIdx.x * 16;
  const int row = r0 + (t >> 4), j = t & 15;

  // State slice first: its latency overlaps the convolution below.
  float* sp = a.state + ((size_t)(h * 128 + row)) * 128 + 8 * j;
  const float4 s_lo = reinterpret_cast<const float4*>(sp)[0];
  const float4 s_hi = reinterpret_cast<const float4*>(sp)[1];

  // Q (threads 0..127) and K (128..255) channels of head h; threads 0..15
  // also own the V channels of this block's rows.
  const int c = t < 128 ? h * 128 + t : 2048 + h * 128 + (t - 128);
  RingTaps rt, rv;
  ring_load(a.ring, a.conv_w, c, rt);
  const int cv = 4096 + h * 128 + r0 + (t & 15);
  if (t < 16) ring_load(a.ring, a.conv_w, cv, rv);
  const int pos = load_pos(a.st, a.pos_val);
  const float v = conv_silu(rt, pos);
  const float ss = tree64(v * v);
  if (lane == 0) red[wave] = ss;
  if (t < 16) {
    const float vval = conv_silu(rv, pos);
    vv[t] = vval;
    if (a.qkv_out) a.qkv_out[cv] = (uint16_t)f2bf(vval);
  }
  if (t == 64) {
    const float ax = rbf(bf2f(a.ab[h]) + bf2f(a.dt_bias[h]));
    const float g = es_exp(-es_exp(a.a_log[h]) * softplus_bf(ax));
    const float beta = sigmoid_bf(bf2f(a.ab[16 + h]));
    gates[0] = g;
    gates[1] = beta;
    if (blockIdx.x == 0) {
      if (a.g_out) a.g_out[h] = g;
      if (a.beta_out) a.beta_out[h] = (uint16_t)f2bf(beta);
    }
  }
  __syncthreads();
  {
    const float tot = t < 128 ? red[0] + red[1] : red[2] + red[3];
    const float inv = 1.0f / sqrtf(tot / 128.0f + 1.0e-6f / 128.0f);
    const float scale = t < 128 ? 0.0078125f : rbf(0.08838834764831845f);
    const float qkv = rbf(rbf(v * inv) * scale);
    qk[t] = qkv;
    if (a.qkv_out && blockIdx.x == 0) a.qkv_out[c] = (uint16_t)f2bf(qkv);
  }
  __syncthreads();

  const float g = gates[0], beta = gates[1];
  float S[8] = {s_lo.x, s_lo.y, s_lo.z, s_lo.w, s_hi.x, s_hi.y, s_hi.z, s_hi.w};
  float kk[8], qq[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    kk[i] = qk[128 + 8 * j + i];
    qq[i] = qk[8 * j + i];
  }
  float mem = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    S[i] = S[i] * g;
    mem = fmaf(S[i], kk[i], mem);
  }
  mem = tree16(mem);
  const float delta = (vv[t >> 4] - mem) * beta;
  float out = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    S[i] = fmaf(kk[i], delta, S[i]);
    out = fmaf(S[i], qq[i], out);
  }
  out = tree16(out);
  if (j == 0) a.y[h * 128 + row] = (uint16_t)f2bf(out);
  reinterpret_cast<float4*>(sp)[0] = make_float4(S[0], S[1], S[2], S[3]);
  reinterpret_cast<float4*>(sp)[1] = make_float4(S[4], S[5], S[6], S[7]);
}

// Recurrence + gated RMSNorm + the head's share of out_proj, one launch per
// layer for the engine. Grid: 16 heads x 8 row-groups (block id = 16 rg + h,
// so a head's blocks share an XCD and its state is read once into that XCD's
// L2), 512 threads. Every
// block runs the whole head's recurrence (its 128 value rows, 4 passes of 32
// rows, 16 lanes per row and 8 keys per lane, the same arithmetic and order as
// k_gdn_recur) so it holds all 128 readouts, writes back only its own 16 state
// rows (all blocks compute the same values), forms the gated norm of the head
// (gdn.metal:238-254, 8 channels per lane, tree16) and the out_proj partial of
// output rows 128*rg .. +127 over the head's 128 columns: per row the four
// 32-column slice partials of k_gdn_gate_out combined by tree4. Because the
// 64-slice tree of a K=2048 row pairs adjacent slices first, the row's full
// sum is the pairwise tree16 of these 16 head partials, formed by the next
// launch, bit for bit.
__global__ __launch_bounds__(512) void k_gdn_recur_out(GdnOutArgs a) {
  __shared__ float qk[256];
  __shared__ float vv[128];
  __shared__ float red[4];
  __shared__ float gates[2];
  __shared__ float yv[128];
  __shared__ float xg[128 + 4];  // gated output, slice s at xg[33 s ..]
  __shared__ float ginv;
  const GdnRecurArgs& r = a.r;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int h = blockIdx.x, rg = blockIdx.y;
  const int j = t & 15;

  // ---- loads, in the order they are needed (loads complete in issue
  // order): conv taps and gate inputs for the prologue, then the state of 4
  // rows per thread, z and the norm weight, then the out_proj slice
  const int pos = load_pos(r.st, r.pos_val);
  // conv channels: q (t < 128), k (t < 256), v (t < 384)
  const int c = t < 128 ? h * 128 + t : t < 256 ? 2048 + h * 128 + (t - 128) : 4096 + h * 128 + (t - 256);
  RingTaps rt;
  if (t < 384) ring_load(r.ring, r.conv_w, c, rt);
  uint32_t ga = 0u, gd = 0u, gb = 0u;
  float gl = 0.0f;
  if (t == 384) {
    ga = r.ab[h];
    gd = r.dt_bias[h];
    gl = r.a_log[h];
    gb = r.ab[16 + h];
  }
  issue_fence();
  float S[4][8];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float* sp = r.state + ((size_t)(h * 128 + p * 32 + (t >> 4))) * 128 + 8 * j;
    const float4 lo = reinterpret_cast<const float4*>(sp)[0];
    const float4 hi = reinterpret_cast<const float4*>(sp)[1];
    S[p][0] = lo.x; S[p][1] = lo.y; S[p][2] = lo.z; S[p][3] = lo.w;
    S[p][4] = hi.x; S[p][5] = hi.y; S[p][6] = hi.z; S[p][7] = hi.w;
  }
  // gated norm inputs: element t (t < 128) of z and of the norm weight
  uint32_t zb = 0u, wb = 0u;
  if (t < 128) {
    zb = a.z[h * 128 + t];
    wb = a.norm_w[t];
  }
  const int orow = rg * 128 + (t >> 2), osl = 4 * h + (t & 3);  // output row, K slice
  const u32x4 oc = *reinterpret_cast<const u32x4*>(a.out.w + (size_t)orow * 256 + osl * 4);
  const uint32_t osv = a.out.s[(size_t)orow * 32 + osl / 2];
  const uint32_t obv = a.out.b[(size_t)orow * 32 + osl / 2];
  issue_fence();

  // ---- conv + SiLU, q/k L2 norm, gates (as k_gdn_recur)
  float v = 0.0f;
  if (t < 384) v = conv_silu(rt, pos);
  if (t < 256) {
    const float ss = tree64(v * v);
    if (lane == 0) red[wave] = ss;
  } else if (t < 384) {
    vv[t - 256] = v;
  } else if (t == 384) {
    const float ax = rbf(bf2f(ga) + bf2f(gd));
    gates[0] = es_exp(-es_exp(gl) * softplus_bf(ax));
    gates[1] = sigmoid_bf(bf2f(gb));
  }
  __syncthreads();
  if (t < 256) {
    const float tot = t < 128 ? red[0] + red[1] : red[2] + red[3];
    const float inv = 1.0f / sqrtf(tot / 128.0f + 1.0e-6f / 128.0f);
    const float scale = t < 128 ? 0.0078125f : rbf(0.08838834764831845f);
    qk[t] = rbf(rbf(v * inv) * scale);
  }
  __syncthreads();

  // ---- recurrence of the head's 128 value rows
  const float g = gates[0], beta = gates[1];
  float kk[8], qq[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    kk[i] = qk[128 + 8 * j + i];
    qq[i] = qk[8 * j + i];
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int row = p * 32 + (t >> 4);
    float mem = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      S[p][i] = S[p][i] * g;
      mem = fmaf(S[p][i], kk[i], mem);
    }
    mem = tree16(mem);
    const float delta = (vv[row] - mem) * beta;
    float out = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      S[p][i] = fmaf(kk[i], delta, S[p][i]);
      out = fmaf(S[p][i], qq[i], out);
    }
    out = tree16(out);
    if (j == 0) yv[row] = bf2f(f2bf(out));
    if ((row >> 4) == rg) {
      float* sp = r.state + ((size_t)(h * 128 + row)) * 128 + 8 * j;
      reinterpret_cast<float4*>(sp)[0] = make_float4(S[p][0], S[p][1], S[p][2], S[p][3]);
      reinterpret_cast<float4*>(sp)[1] = make_float4(S[p][4], S[p][5], S[p][6], S[p][7]);
    }
  }
  __syncthreads();

  // ---- gated RMSNorm of the head (as k_gdn_gate_out): sum of squares as 16
  // lanes x 8 channels (fma chain, tree16), then one channel per thread
  if (t < 16) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(yv[t * 8 + i], yv[t * 8 + i], ss);
    ss = tree16(ss);
    if (t == 0) ginv = 1.0f / sqrtf(ss / 128.0f + 1e-6f);
  }
  __syncthreads();
  if (t < 128) {
    const float norm = rbf(rbf(yv[t] * ginv) * bf2f(wb));
    const float gz = bf2f(zb);
    const float sy = 1.0f / (1.0f + es_exp(fabsf(gz)));
    const float sig = gz < 0.0f ? sy : 1.0f - sy;
    xg[t + (t >> 5)] = rbf((gz * sig) * norm);
  }
  __syncthreads();

  // ---- out_proj partial: 4 lanes per output row, one 32-column slice each
  float xv[32], xr[32];
  const int sl = t & 3;
#pragma unroll
  for (int q = 0; q < 32; ++q) xv[q] = xg[sl * 33 + q];
  const float xs = prep_slice(xv, xr);
  const float part = tree4(q4_slice(oc, osv, obv, xr, xs));
  if (sl == 0) a.part[(size_t)h * 1024 + orow] = part;
}

}  // namespace

hipError_t launch_gdn_recur(const GdnRecurArgs& a, hipStream_t s) {
  if (!a.ring || !a.conv_w || !a.ab || !a.a_log || !a.dt_bias || !a.state || !a.y)
    return hipErrorInvalidValue;
  if (!a.st && a.pos_val < 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gdn_recur, dim3(8, kGdnHeads), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_gdn_recur_out(const GdnOutArgs& a, hipStream_t s) {
  const GdnRecurArgs& r = a.r;
  if (!r.ring || !r.conv_w || !r.ab || !r.a_log || !r.dt_bias || !r.state || !a.z || !a.norm_w ||
      !a.part || !a.out.w || !a.out.s || !a.out.b || a.out.n != kHidden || a.out.k != 2048)
    return hipErrorInvalidValue;
  if (!r.st && r.pos_val < 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gdn_recur_out, dim3(kGdnHeads, 8), dim3(512), 0, s, a);
  return hipGetLastError();
}

}  // namespace es
