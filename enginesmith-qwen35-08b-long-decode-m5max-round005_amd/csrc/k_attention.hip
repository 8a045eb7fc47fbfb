// GQA decode attention on gfx950 (8 query heads, 2 KV heads, head dim 256,
// one query token), computing the reference's own two routes
// (model.rs:327-347) in a fixed fp32 order:
//   length < 1024: 32 position chains (chain c takes positions c, c+32, ...),
//     combined in fp32 (sdpa_vector, attention_decode.metal:51-213);
//   length >= 1024: 64 chains whose unnormalised outputs are rounded to bf16,
//     then merged and gated (sdpa_vector_2pass_1 + attn_decode_split2_gate,
//     attention_decode.metal:215-431, 830-891).
//
// k_attn_scores, grid (blocks, 2 KV heads) x 256: the prologue fuses
//   attn_prepare_qkv_decode (attention.metal:262-313: q/k RMSNorm with bf16
//   normalised value and bf16 gain product, RoPE on dims 0..63 with pairs
//   (i, i+32)); the block whose chunk holds the new position also writes its
//   K/V rows. Each block then streams a contiguous chunk of the K cache once
//   for all four query heads of the group: 8 lanes per position, lane m holds
//   dims 8m+64i .. +7 (i = 0..3, 128 coalesced bytes per 8 lanes), one fma
//   chain per 8 dims, (p[m]+p[m+8])+(p[m+16]+p[m+24]) in the lane and a DPP
//   tree over the 8 lanes. Scores go to an fp32 array [8, capacity].
// k_attn_chain, 256 blocks x 320 threads: block = (KV head, chain, query-head
//   pair). Waves 0..3 own one value dim each for both heads; wave 4 turns the
//   chain's scores into running max, factor and exp score, 64 steps at a time
//   and one tile ahead (max scan by DPP, exp by the shared series). Per step
//   o = fma(e, v, o*factor) and sum = sum*factor + e; when every factor of a
//   tile is exactly 1 the products by 1 are skipped, which changes no bit.
//   The two blocks of a (KV head, chain) sit on the same XCD (block ids b and
//   b+8) so the second read of each V row is an L2 hit.
// k_attn_merge, grid (8 heads, 4 quarters) x 64: chain combination of either
//   route, then gated = bf16(bf16(o) * sigmoid_bf(gate)) (attention.metal:133-151).
#include "es_kernels.hpp"

namespace es {
namespace {

constexpr float kFiniteMin = -3.40282346638528859812e38f;

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

__device__ __forceinline__ float tree8(float v) {
  v = tree4(v);
  return v + dpp_half_mirror(v);
}

// fma chain over the 8 bf16 dims of one 16-byte K chunk.
__device__ __forceinline__ float chunk_dot(const float* q, const u32x4& k) {
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    s = fmaf(q[2 * w], bf_lo(k[w]), s);
    s = fmaf(q[2 * w + 1], bf_hi(k[w]), s);
  }
  return s;
}

__global__ __launch_bounds__(256, 2) void k_attn_scores(AttnArgs a) {
  __shared__ float nrm[5][256];     // normalised q heads 0..3, new k
  __shared__ float qs[4][256];      // roped q * 1/16
  __shared__ u32x4 knew[32];        // new K row (roped, bf16)

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int g = blockIdx.y, B = gridDim.x;
  const int pos = load_pos(a.st, a.pos_val);
  const int n = pos + 1;
  int chunk = (n + B - 1) / B;
  chunk = (chunk + 31) & ~31;
  const int start = blockIdx.x * chunk;
  if (start >= n) return;
  const int end = min(start + chunk, n);
  const bool owner = end == n;  // this chunk holds the new position

  const int grp = lane >> 3, m = lane & 7;
  const uint16_t* kb = a.kcache + (size_t)g * a.capacity * 256 + 8 * m;
  // First K rows, issued before the prologue so their latency overlaps it.
  u32x4 kc[4] = {}, kn[4] = {};
  int p = start + wave * 8 + grp;
  if (p < end && p != pos) {
    const u32x4* r = reinterpret_cast<const u32x4*>(kb + (size_t)p * 256);
#pragma unroll
    for (int i = 0; i < 4; ++i) kc[i] = r[8 * i];
  }

  // ---- prologue: q (and, in the owner block, the new k/v rows) ----
  {
    float o4[4];
    head_norm4(a.q_proj + (4 * g + wave) * 512, a.q_gain, lane, o4);
#pragma unroll
    for (int i = 0; i < 4; ++i) nrm[wave][lane * 4 + i] = o4[i];
    if (owner && wave == 0) {
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
    if (a.query_out && blockIdx.x == 0) {
      uint16_t* qo = a.query_out + (4 * g + wave) * 256 + lane * 4;
      *reinterpret_cast<uint2*>(qo) = make_uint2(pack_bf2(r[0], r[1]), pack_bf2(r[2], r[3]));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) qs[wave][lane * 4 + i] = r[i] * 0.0625f;
    if (owner && wave == 1) {
      float kr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) kr[i] = rope_at(nrm[4], lane * 4 + i, pos, a.inv_freq);
      const uint32_t k0 = pack_bf2(kr[0], kr[1]);
      const uint32_t k1 = pack_bf2(kr[2], kr[3]);
      uint32_t* kw = reinterpret_cast<uint32_t*>(knew);
      kw[lane * 2] = k0;
      kw[lane * 2 + 1] = k1;
      const size_t ci = ((size_t)g * a.capacity + pos) * 256 + lane * 4;
      *reinterpret_cast<uint2*>(a.kcache + ci) = make_uint2(k0, k1);
      *reinterpret_cast<uint2*>(a.vcache + ci) =
          *reinterpret_cast<const uint2*>(a.v_proj + g * 256 + lane * 4);
    }
  }
  __syncthreads();

  // q for this lane's dims: 4 heads x 4 chunks x 8 dims.
  float q[4][4][8];
#pragma unroll
  for (int hh = 0; hh < 4; ++hh)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) q[hh][i][j] = qs[hh][64 * i + 8 * m + j];

  float* sc = a.scores + (size_t)(4 * g + (m & 3)) * a.capacity;
  for (; p - grp < end; p += 32) {
    const int pn = p + 32;
    if (pn < end && pn != pos) {
      const u32x4* r = reinterpret_cast<const u32x4*>(kb + (size_t)pn * 256);
#pragma unroll
      for (int i = 0; i < 4; ++i) kn[i] = r[8 * i];
    }
    if (p == pos) {
#pragma unroll
      for (int i = 0; i < 4; ++i) kc[i] = knew[m + 8 * i];
    }
    float s[4];
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      const float p0 = chunk_dot(q[hh][0], kc[0]);
      const float p1 = chunk_dot(q[hh][1], kc[1]);
      const float p2 = chunk_dot(q[hh][2], kc[2]);
      const float p3 = chunk_dot(q[hh][3], kc[3]);
      s[hh] = tree8((p0 + p1) + (p2 + p3));
    }
    const int hm = m & 3;
    const float mine = hm == 0 ? s[0] : hm == 1 ? s[1] : hm == 2 ? s[2] : s[3];
    if (p < end && m < 4) sc[p] = mine;
#pragma unroll
    for (int i = 0; i < 4; ++i) kc[i] = kn[i];
  }
}

// ---- per-chain online softmax ----

constexpr int kTile = 64;

template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_src(float x, float old) {
  return __builtin_amdgcn_update_dpp(old, x, CTRL, ROWS, 0xf, false);
}

// Inclusive max scan over the 64 lanes (GFX9 row_shr and row_bcast DPP).
__device__ __forceinline__ float wave_max_scan(float x) {
  const float ninf = -__builtin_inff();
  x = fmaxf(x, dpp_src<0x111, 0xf>(x, ninf));  // row_shr:1
  x = fmaxf(x, dpp_src<0x112, 0xf>(x, ninf));  // row_shr:2
  x = fmaxf(x, dpp_src<0x114, 0xf>(x, ninf));  // row_shr:4
  x = fmaxf(x, dpp_src<0x118, 0xf>(x, ninf));  // row_shr:8
  x = fmaxf(x, dpp_src<0x142, 0xa>(x, ninf));  // row_bcast:15 into rows 1, 3
  x = fmaxf(x, dpp_src<0x143, 0xc>(x, ninf));  // row_bcast:31 into rows 2, 3
  return x;
}

__device__ __forceinline__ float readlane63(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

// Exp scores and factors of one tile for both heads of the block.
struct ChainTile {
  float e[2][kTile];
  float f[2][kTile];
  int slow;  // some factor of the tile differs from 1
};

// Raw bf16 V values of one tile through a buffer resource based at the
// chain's first row: the row offset is a scalar, the lane's dim the vector
// offset, so no address arithmetic runs per load. Rows past the chain's end
// re-read its last row (in bounds; their e is 0), so the loads carry no
// branches and all 64 stay in flight until their first use. Requires L >= 1.
__device__ __forceinline__ void load_tile(__amdgpu_buffer_rsrc_t vb, uint32_t voff,
                                          uint32_t row_bytes, int j0, int L, uint32_t* v) {
#pragma unroll
  for (int s = 0; s < kTile; ++s)
    v[s] = __builtin_amdgcn_raw_buffer_load_b16(vb, voff, (uint32_t)min(j0 + s, L - 1) * row_bytes, 0);
}

__device__ __forceinline__ float v_f32(uint32_t raw) { return __builtin_bit_cast(float, raw << 16); }

// One tile of 64 steps for the dim owned by this thread; WS selects the head
// whose sum this wave keeps. Steps past the chain's end have e = 0 and f = 1
// and change nothing (o is never -0, v is finite).
template <bool SLOW, int WS>
__device__ __forceinline__ void chain_tile(const ChainTile& T, const uint32_t* raw, float& o0,
                                           float& o1, float& sum) {
#pragma unroll
  for (int s = 0; s < kTile; ++s) {
    const float e0 = T.e[0][s], e1 = T.e[1][s];
    const float v = v_f32(raw[s]);
    const float es = WS ? e1 : e0;
    if (SLOW) {
      o0 = fmaf(e0, v, o0 * T.f[0][s]);
      o1 = fmaf(e1, v, o1 * T.f[1][s]);
      sum = sum * T.f[WS][s] + es;
    } else {
      o0 = fmaf(e0, v, o0);
      o1 = fmaf(e1, v, o1);
      sum = sum + es;
    }
  }
}

template <int WS>
__device__ __forceinline__ void run_tile(const ChainTile& T, const uint32_t* v, float& o0, float& o1,
                                         float& sum) {
  if (T.slow)
    chain_tile<true, WS>(T, v, o0, o1, sum);
  else
    chain_tile<false, WS>(T, v, o0, o1, sum);
}

template <int WS>
__device__ __forceinline__ void dims_loop(const ChainTile* tiles, __amdgpu_buffer_rsrc_t vb,
                                          uint32_t voff, uint32_t stride, int L, float& o0,
                                          float& o1, float& sum) {
  if (L == 0) return;
  uint32_t va[kTile], vn[kTile];
  load_tile(vb, voff, stride, 0, L, va);
  for (int j0 = 0, k = 0; j0 < L; j0 += 2 * kTile, k += 2) {
    load_tile(vb, voff, stride, j0 + kTile, L, vn);
    __syncthreads();
    run_tile<WS>(tiles[k & 1], va, o0, o1, sum);
    if (j0 + kTile >= L) break;
    load_tile(vb, voff, stride, j0 + 2 * kTile, L, va);
    __syncthreads();
    run_tile<WS>(tiles[(k + 1) & 1], vn, o0, o1, sum);
  }
}

__global__ __launch_bounds__(320, 1) void k_attn_chain(AttnArgs a) {
  __shared__ ChainTile tiles[2];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int bx = blockIdx.x;
  const int hp = (bx >> 3) & 1, rest = (bx & 7) | ((bx >> 4) << 3);
  const int kvh = rest >> 6, c = rest & 63;
  const int pos = load_pos(a.st, a.pos_val);
  const int n = pos + 1;
  const int C = n < kAttnRouteSplit ? 32 : 64;
  if (c >= C) return;
  const int L = n > c ? (n - 1 - c) / C + 1 : 0;
  const int h0 = 4 * kvh + 2 * hp;

  if (wave == 4) {
    // Lane = step within a tile, both heads; one tile ahead of the dim waves.
    const float* sc0 = a.scores + (size_t)h0 * a.capacity + c;
    const float* sc1 = sc0 + a.capacity;
    const float ninf = -__builtin_inff();
    float m0 = kFiniteMin, m1 = kFiniteMin;
    float s0 = lane < L ? sc0[(size_t)lane * C] : ninf;
    float s1 = lane < L ? sc1[(size_t)lane * C] : ninf;
    for (int j0 = 0, k = 0; j0 < L; j0 += kTile, ++k) {
      const int jn = j0 + kTile + lane;
      const float s0n = jn < L ? sc0[(size_t)jn * C] : ninf;
      const float s1n = jn < L ? sc1[(size_t)jn * C] : ninf;
      const float mt0 = fmaxf(m0, wave_max_scan(s0));
      const float mt1 = fmaxf(m1, wave_max_scan(s1));
      const float pv0 = dpp_src<0x138, 0xf>(mt0, m0);  // wave_shr:1, lane 0 <- carry
      const float pv1 = dpp_src<0x138, 0xf>(mt1, m1);
      const float f0 = es_exp(pv0 - mt0), e0 = es_exp(s0 - mt0);
      const float f1 = es_exp(pv1 - mt1), e1 = es_exp(s1 - mt1);
      ChainTile& T = tiles[k & 1];
      T.e[0][lane] = e0;
      T.e[1][lane] = e1;
      T.f[0][lane] = f0;
      T.f[1][lane] = f1;
      const bool slow = __any(f0 != 1.0f || f1 != 1.0f);
      if (lane == 0) T.slow = slow;
      m0 = readlane63(mt0);
      m1 = readlane63(mt1);
      s0 = s0n;
      s1 = s1n;
      __syncthreads();
    }
    if (lane == 0) {
      a.part_ml[((size_t)h0 * kAttnMaxChains + c) * 2] = m0;
      a.part_ml[((size_t)(h0 + 1) * kAttnMaxChains + c) * 2] = m1;
    }
    return;
  }

  // Buffer over this KV head's rows from the chain's first row to the end.
  const __amdgpu_buffer_rsrc_t vb = __builtin_amdgcn_make_buffer_rsrc(
      a.vcache + ((size_t)kvh * a.capacity + c) * 256, 0, (a.capacity - c) * 512, 0x00020000);
  const uint32_t stride = (uint32_t)C * 512;
  float o0 = 0.0f, o1 = 0.0f, sum = 0.0f;
  if (wave & 1)
    dims_loop<1>(tiles, vb, (uint32_t)t * 2, stride, L, o0, o1, sum);
  else
    dims_loop<0>(tiles, vb, (uint32_t)t * 2, stride, L, o0, o1, sum);
  a.part_o[((size_t)h0 * kAttnMaxChains + c) * 256 + t] = o0;
  a.part_o[((size_t)(h0 + 1) * kAttnMaxChains + c) * 256 + t] = o1;
  if (wave < 2 && lane == 0)
    a.part_ml[((size_t)(h0 + wave) * kAttnMaxChains + c) * 2 + 1] = sum;
}

// ---- merge + gate ----

// Pairwise sum of 32 values in index order.
__device__ __forceinline__ float tree_reg32(float* v) {
#pragma unroll
  for (int off = 1; off < 32; off *= 2)
#pragma unroll
    for (int i = 0; i + off < 32; i += 2 * off) v[i] = v[i] + v[i + off];
  return v[0];
}

__global__ __launch_bounds__(64) void k_attn_merge(AttnArgs a) {
  __shared__ float fac[kAttnMaxChains];
  __shared__ float total;
  const int lane = threadIdx.x, h = blockIdx.x;
  const int d = blockIdx.y * 64 + lane;
  const int pos = load_pos(a.st, a.pos_val);
  const bool two_pass = pos + 1 >= kAttnRouteSplit;
  const float* ml = a.part_ml + (size_t)h * kAttnMaxChains * 2;
  const float* po = a.part_o + (size_t)h * kAttnMaxChains * 256 + d;
  float v[kAttnMaxChains];
  // Chain outputs first: independent loads in flight while the factors form.
#pragma unroll
  for (int c = 0; c < 32; ++c) v[c] = po[(size_t)c * 256];
  if (two_pass) {
#pragma unroll
    for (int c = 32; c < 64; ++c) v[c] = po[(size_t)c * 256];
    const float mx = ml[2 * lane];
    const float F = es_exp(mx - wave_max(mx));
    fac[lane] = F;
    // lane l < 32: (0 + F_l s_l) + F_{l+32} s_{l+32}, then pairwise over lanes
    // (attention_decode.metal:858-862).
    const float prod = F * ml[2 * lane + 1];
    const float hi = __shfl_down(prod, 32, 64);
    float s = 0.0f;
    s = s + prod;
    s = s + hi;
    s = tree32(s);
    if (lane == 0) total = s;
  } else {
    const float mx = lane < 32 ? ml[2 * lane] : kFiniteMin;
    const float F = es_exp(mx - wave_max(mx));
    if (lane < 32) fac[lane] = F;
    const float s = tree32(ml[2 * (lane & 31) + 1] * F);
    if (lane == 0) total = s;
  }
  __syncthreads();
  const float sum = total;
  float o;
  if (two_pass) {
    float w[32];
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      float acc = 0.0f;
      acc = acc + fac[l] * rbf(v[l]);
      acc = acc + fac[l + 32] * rbf(v[l + 32]);
      w[l] = acc;
    }
    o = tree_reg32(w);
  } else {
#pragma unroll
    for (int l = 0; l < 32; ++l) v[l] = v[l] * fac[l];
    o = tree_reg32(v);
  }
  o = sum == 0.0f ? o : o / sum;
  const float attention = rbf(o);
  const float gate = sigmoid_bf(bf2f(a.q_proj[h * 512 + 256 + d]));
  a.gated[h * 256 + d] = (uint16_t)f2bf(attention * gate);
}

bool attn_ok(const AttnArgs& a) {
  return a.q_proj && a.k_proj && a.v_proj && a.q_gain && a.k_gain && a.kcache && a.vcache &&
         a.inv_freq && a.part_o && a.part_ml && a.scores && a.gated && a.blocks >= 1 &&
         a.blocks <= 1024 && a.capacity > 0 &&
         (a.st || (a.pos_val >= 0 && a.pos_val < a.capacity));
}

}  // namespace

size_t attn_scratch_bytes(int capacity) {
  return ((size_t)kQHeads * kAttnMaxChains * (256 + 2) + (size_t)kQHeads * capacity) *
         sizeof(float);
}

void attn_bind_scratch(AttnArgs& a, void* scratch) {
  a.part_o = static_cast<float*>(scratch);
  a.part_ml = a.part_o + (size_t)kQHeads * kAttnMaxChains * 256;
  a.scores = a.part_ml + (size_t)kQHeads * kAttnMaxChains * 2;
}

hipError_t launch_attn_scores(const AttnArgs& a, hipStream_t s) {
  if (!attn_ok(a)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_scores, dim3(a.blocks, kKvHeads), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_attn_chain(const AttnArgs& a, hipStream_t s) {
  if (!attn_ok(a)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_chain, dim3(kKvHeads * kAttnMaxChains * 2), dim3(320), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_attn_merge(const AttnArgs& a, hipStream_t s) {
  if (!attn_ok(a)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_merge, dim3(kQHeads, 4), dim3(64), 0, s, a);
  return hipGetLastError();
}

}  // namespace es
