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
// k_attn_chain, 256 blocks x 448 threads: block = (KV head, chain, query-head
//   pair), thread = two adjacent value dims of one head (four compute waves),
//   plus one data-moving wave and one exps wave per head. V rows and scores
//   are staged in
//   LDS by 16-byte global->LDS DMA, four 64-step tiles deep. The exps waves
//   turn the chain's scores into running max, factor and exp score one tile ahead
//   (max scan by DPP, exp by the shared series), which reach the compute
//   lanes by DPP row broadcast. Per step o = fma(e, v, o*factor)
//   and sum = sum*factor + e; when every factor of a tile is exactly 1 the
//   products by 1 are skipped, which changes no bit.
//   The two blocks of a (KV head, chain) sit on the same XCD (block ids b and
//   b+8) so the second read of each V row is an L2 hit.
// k_attn_merge, grid (8 heads, 4 quarters) x 64: chain combination of either
//   route, then gated = bf16(bf16(o) * sigmoid_bf(gate)) (attention.metal:133-151).
#include "es_kernels.hpp"

namespace es {
namespace {

constexpr float kFiniteMin = -3.40282346638528859812e38f;

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
// d < 32: fma(lo, c, -(hi*s)); 32 <= d < 64: fma(lo, s, hi*c).
// inv is inv_freq[d & 31] (read by the caller, only used for d < 64).
__device__ __forceinline__ float rope_at(const float* nrm, int d, int pos, float inv) {
  if (d >= 64) return nrm[d];
  const int pair = d & 31;
  const float angle = (float)pos * inv;
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

// Row stride of the score array: j-slots per chain, for the 32-chain route,
// rounded up to whole 64-step tiles.
__host__ __device__ __forceinline__ int score_stride(int capacity) {
  return (((capacity + 31) / 32) + 63) & ~63;
}

__device__ __forceinline__ int route_chains(int n) { return n < kAttnRouteSplit ? 32 : 64; }

constexpr int kRing = 4;  // K-row register slots per lane in k_attn_scores

__global__ __launch_bounds__(256, 2) void k_attn_scores(AttnArgs a) {
  __shared__ float nrm[5][256];     // normalised q heads 0..3, new k
  __shared__ float qs[4][256];      // roped q * 1/16
  __shared__ u32x4 knew[32];        // new K row (roped, bf16)

  // wave is uniform; readfirstlane lets the compiler keep the item loop scalar.
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int g = blockIdx.y, B = gridDim.x;
  const int pos = load_pos(a.st, a.pos_val);
  const int n = pos + 1;
  const int C = route_chains(n);
  // Work items (chain c, 8 steps from 8*j8): item i = j8*C + c covers
  // positions c + C*(8*j8 + r), r = 0..7. Block b owns items [ib0, ib1).
  const int jtot = (n + C - 1) / C;
  const int items = C * ((jtot + 7) >> 3);
  const int ipb = (items + B - 1) / B;
  const int ib0 = blockIdx.x * ipb;
  if (ib0 >= items) return;
  const int ib1 = min(ib0 + ipb, items);
  const int ipos = (pos / C >> 3) * C + pos % C;
  const bool owner = ib0 <= ipos && ipos < ib1;  // holds the new position
  const int grp = lane >> 3, m = lane & 7;
  const uint16_t* kb = a.kcache + (size_t)g * a.capacity * 256 + 8 * m;
  // Lane group grp takes step r = grp of the item; wave w takes items
  // ib0 + w, ib0 + w + 4, ...
  const int lc = C == 32 ? 5 : 6;  // log2 C
  auto item_pos = [&](int i, int& p) {
    p = (i & (C - 1)) + ((8 * (i >> lc) + grp) << lc);
    return p < n;
  };
  // Prologue inputs, read before the K ring so that waiting for them does not
  // wait for K (vector-memory counters complete in order).
  const uint2 qx = *reinterpret_cast<const uint2*>(a.q_proj + (4 * g + wave) * 512 + lane * 4);
  const uint2 qg = *reinterpret_cast<const uint2*>(a.q_gain + lane * 4);
  const uint2 kx = *reinterpret_cast<const uint2*>(a.k_proj + g * 256 + lane * 4);
  const uint2 kg = *reinterpret_cast<const uint2*>(a.k_gain + lane * 4);
  const uint2 vx = *reinterpret_cast<const uint2*>(a.v_proj + g * 256 + lane * 4);
  float inv[4];
#pragma unroll
  for (int x = 0; x < 4; ++x) inv[x] = a.inv_freq[((lane * 4) & 31) + x];
  // Wave w takes items ib0 + w + 4*it, it = 0 .. nit-1. K rows stream
  // through a ring of kRing register slots, kRing - 1 items in flight while
  // one is computed; the first kRing - 1 are issued before the prologue so
  // their latency overlaps it. Loads are unconditional: an item past the end
  // reads row 0 and the new position's row (written by this kernel) is read
  // but replaced by the LDS copy, so no branch holds a load back.
  const int nit = ib1 - ib0 > wave ? (ib1 - ib0 - wave + 3) / 4 : 0;
  u32x4 kr[kRing][4];
  int pr[kRing];
  bool okr[kRing];
  auto issue = [&](int it, u32x4* dst, int& pp, bool& okk) {
    okk = it < nit && item_pos(ib0 + wave + 4 * it, pp);
    const u32x4* r = reinterpret_cast<const u32x4*>(kb + (size_t)(okk ? pp : 0) * 256);
#pragma unroll
    for (int x = 0; x < 4; ++x) dst[x] = r[8 * x];
  };
#pragma unroll
  for (int u = 0; u < kRing - 1; ++u) issue(u, kr[u], pr[u], okr[u]);

  // ---- prologue: q (and, in the owner block, the new k/v rows) ----
  {
    float o4[4];
    head_norm4(qx, qg, o4);
#pragma unroll
    for (int x = 0; x < 4; ++x) nrm[wave][lane * 4 + x] = o4[x];
    if (owner && wave == 0) {
      head_norm4(kx, kg, o4);
#pragma unroll
      for (int x = 0; x < 4; ++x) nrm[4][lane * 4 + x] = o4[x];
    }
  }
  __syncthreads();
  {
    float r[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) r[x] = rope_at(nrm[wave], lane * 4 + x, pos, inv[x]);
    if (a.query_out && blockIdx.x == 0) {
      uint16_t* qo = a.query_out + (4 * g + wave) * 256 + lane * 4;
      *reinterpret_cast<uint2*>(qo) = make_uint2(pack_bf2(r[0], r[1]), pack_bf2(r[2], r[3]));
    }
#pragma unroll
    for (int x = 0; x < 4; ++x) qs[wave][lane * 4 + x] = r[x] * 0.0625f;
    if (owner && wave == 1) {
      float kr[4];
#pragma unroll
      for (int x = 0; x < 4; ++x) kr[x] = rope_at(nrm[4], lane * 4 + x, pos, inv[x]);
      const uint32_t k0 = pack_bf2(kr[0], kr[1]);
      const uint32_t k1 = pack_bf2(kr[2], kr[3]);
      uint32_t* kw = reinterpret_cast<uint32_t*>(knew);
      kw[lane * 2] = k0;
      kw[lane * 2 + 1] = k1;
      const size_t ci = ((size_t)g * a.capacity + pos) * 256 + lane * 4;
      *reinterpret_cast<uint2*>(a.kcache + ci) = make_uint2(k0, k1);
      *reinterpret_cast<uint2*>(a.vcache + ci) = vx;
    }
  }
  __syncthreads();

  // q for this lane's dims: 4 heads x 4 chunks x 8 dims.
  float q[4][4][8];
#pragma unroll
  for (int hh = 0; hh < 4; ++hh)
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int j = 0; j < 8; ++j) q[hh][x][j] = qs[hh][64 * x + 8 * m + j];

  const int sstride = score_stride(a.capacity);
  float* sc = a.scores + (size_t)(4 * g + (m & 3)) * kAttnMaxChains * sstride;
  for (int it0 = 0; it0 < nit; it0 += kRing) {
#pragma unroll
    for (int u = 0; u < kRing; ++u) {
      const int it = it0 + u;  // items past nit compute on row 0 and store nothing
      const int nx = (u + kRing - 1) % kRing;  // slot freed by the previous item
      issue(it + kRing - 1, kr[nx], pr[nx], okr[nx]);
      u32x4 kc[4];
#pragma unroll
      for (int x = 0; x < 4; ++x) kc[x] = okr[u] && pr[u] == pos ? knew[m + 8 * x] : kr[u][x];
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
      const int p = pr[u];
      if (okr[u] && m < 4) sc[(size_t)(p & (C - 1)) * sstride + (p >> lc)] = mine;
    }
  }
}

// ---- per-chain online softmax ----

constexpr int kTile = 64;    // chain steps per tile
constexpr int kStages = 4;   // V tiles in LDS (3 in flight while one is used)

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

struct __attribute__((aligned(16))) ChainSmem {
  uint16_t v[kStages][kTile][256];  // V rows of a tile, as loaded
  float s[kStages][2][kTile];       // scores of a tile, both heads
  float e[2][2][kTile];             // [buffer][head][step] exp scores
  float f[2][2][kTile];             // factors
  int slow[2][2];                   // some factor of the tile differs from 1
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Barrier for LDS written by ds_write and by global->LDS DMA. The caller has
// waited for its own DMA (vmcnt); lgkmcnt(0) covers ds_write. The empty asm
// keeps the compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt and expcnt untouched
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Wait until at most N vector-memory operations of this wave are pending
// (gfx9 encoding: vmcnt[3:0] | expcnt 7 | lgkmcnt 15 | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Issue tile T from the producer wave: 64 V rows as 32 DMA of 1 KB (lanes
// 0..31 one row, 32..63 the next) and the tile's 2 x 64 scores as one DMA of
// 32 x 16 B (33 vector-memory operations). Rows past the chain's end re-read
// its last row (in bounds; their slots are masked by e = 0).
constexpr int kTileOps = 33;
__device__ __forceinline__ void issue_tile(ChainSmem& sm, const uint16_t* vrow0, const float* sc0,
                                           int sstride, int C, int L, int T, int lane) {
  const int st = T % kStages;
#pragma unroll 4
  for (int x = 0; x < 32; ++x) {
    const int r = 2 * x;
    const int j = min(T * kTile + r + (lane >> 5), L - 1);
    const uint16_t* g = vrow0 + (size_t)j * C * 256 + (lane & 31) * 8;
    __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)&sm.v[st][r][0], 16, 0, 0);
  }
  if (lane < 32) {
    const int head = lane >> 4, part = lane & 15;
    const float* g = sc0 + (size_t)head * kAttnMaxChains * sstride + T * kTile + part * 4;
    __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)&sm.s[st][0][0], 16, 0, 0);
  }
}

// Exp scores and factors of tile T for one head from its staged scores.
__device__ __forceinline__ void tile_exps(ChainSmem& sm, int T, int L, int head, int lane,
                                          float& carry) {
  const float ninf = -__builtin_inff();
  const float s = T * kTile + lane < L ? sm.s[T % kStages][head][lane] : ninf;
  const float mt = fmaxf(carry, wave_max_scan(s));
  const float pv = dpp_src<0x138, 0xf>(mt, carry);  // wave_shr:1, lane 0 <- carry
  const float f = es_exp(pv - mt), e = es_exp(s - mt);
  sm.e[T & 1][head][lane] = e;
  sm.f[T & 1][head][lane] = f;
  sm.slow[T & 1][head] = __any(f != 1.0f);  // wave-uniform, stored by every lane
  carry = readlane63(mt);
}

// Exp scores and factors reach the compute waves through DPP: each lane
// holds e[16r + (lane & 15)] for r = 0..3 (one 4-byte LDS read per r), and
// step s = 16r + k uses row_newbcast:k, which gives every lane of a 16-lane
// row the value of that row's lane k, as the first operand of the
// arithmetic. The registers read this way are only ever written by LDS loads,
// so no VALU-write-to-DPP-read wait states are needed.
template <int K>
__device__ __forceinline__ void fmac_bcast(float& acc, float e_row, float v) {
  asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
      : "+v"(acc) : "v"(e_row), "v"(v), "n"(K));
}
template <int K>
__device__ __forceinline__ float mul_bcast(float f_row, float x) {
  float r;
  asm("v_mul_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
      : "=v"(r) : "v"(f_row), "v"(x), "n"(K));
  return r;
}
template <int K>
__device__ __forceinline__ float add_bcast(float e_row, float x) {
  float r;
  asm("v_add_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
      : "=v"(r) : "v"(e_row), "v"(x), "n"(K));
  return r;
}

// One chain step of the two dims (va, vb) owned by this thread, exp score
// and factor of step 16r + K broadcast from er / fr:
// o = fma(e, v, o*f) and sum = sum*f + e, or with f == 1 for the whole tile
// o = fma(e, v, o) and sum = sum + e (products by 1 skipped, same bits).
template <int K, bool SLOW, bool SUM>
__device__ __forceinline__ void chain_step(float er, float fr, float va, float vb, float& oa,
                                           float& ob, float& sum) {
  if (SLOW) {
    oa = mul_bcast<K>(fr, oa);
    ob = mul_bcast<K>(fr, ob);
    if (SUM) sum = mul_bcast<K>(fr, sum);
  }
  fmac_bcast<K>(oa, er, va);
  fmac_bcast<K>(ob, er, vb);
  if (SUM) sum = add_bcast<K>(er, sum);
}

// Eight steps 8g .. 8g+7: the two dims of a step are one dword and the
// loads pair rows 512 B apart into one LDS read (four reads per group).
__device__ __forceinline__ void load_group(const uint32_t* vw, int kw, int g, uint32_t* w) {
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i] = vw[(8 * g + i) * 128 + kw];
}

template <int G, bool SLOW, bool SUM>
__device__ __forceinline__ void chain_group(const uint32_t* w, float er, float fr, float& oa,
                                            float& ob, float& sum) {
  constexpr int k0 = 8 * (G & 1);  // lane of the 16-lane row holding step 8G
#define ES_STEP(I) chain_step<k0 + I, SLOW, SUM>(er, fr, bf_lo(w[I]), bf_hi(w[I]), oa, ob, sum)
  ES_STEP(0); ES_STEP(1); ES_STEP(2); ES_STEP(3); ES_STEP(4); ES_STEP(5); ES_STEP(6); ES_STEP(7);
#undef ES_STEP
}

// Groups G .. 7 of a tile: compute group G, then issue the loads of group
// G + AHEAD into the slot it frees. LDS reads complete in order and at most
// 15 may be outstanding (the counter's width), so a fast tile keeps three
// groups in flight (plus two reads of exp scores) and a slow tile, which also
// reads factors, two.
template <int G, bool SLOW, bool SUM>
__device__ __forceinline__ void chain_groups(const uint32_t* vw, int kw, const float* er,
                                             const float* fr, uint32_t (&w)[4][8], float& oa,
                                             float& ob, float& sum) {
  if constexpr (G < 8) {
    constexpr int ahead = SLOW ? 2 : 3;
    chain_group<G, SLOW, SUM>(w[G % 4], er[G / 2], fr[G / 2], oa, ob, sum);
    issue_fence();
    if constexpr (G + ahead < 8) {
      load_group(vw, kw, G + ahead, w[(G + ahead) % 4]);
      issue_fence();
    }
    chain_groups<G + 1, SLOW, SUM>(vw, kw, er, fr, w, oa, ob, sum);
  }
}

// 64 steps of the two adjacent dims owned by this thread for one head; SUM
// waves also keep the head's sum. Steps past the chain's end have e = 0 and
// f = 1 and change nothing (o is never -0, V rows are finite).
template <bool SLOW, bool SUM>
__device__ __forceinline__ void chain_tile(const ChainSmem& sm, int T, int hh, int kw, int lane,
                                           float& oa, float& ob, float& sum) {
  const int st = T % kStages, b = T & 1;
  const uint32_t* vw = reinterpret_cast<const uint32_t*>(&sm.v[st][0][0]);
  const float* ep = sm.e[b][hh] + (lane & 15);
  const float* fp = sm.f[b][hh] + (lane & 15);
  float er[4], fr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    er[r] = ep[16 * r];
    fr[r] = SLOW ? fp[16 * r] : 1.0f;
  }
  issue_fence();
  uint32_t w[4][8];
  constexpr int ahead = SLOW ? 2 : 3;
#pragma unroll
  for (int g = 0; g < ahead; ++g) load_group(vw, kw, g, w[g]);
  issue_fence();
  chain_groups<0, SLOW, SUM>(vw, kw, er, fr, w, oa, ob, sum);
}

template <bool SUM>
__device__ __forceinline__ void run_tile(const ChainSmem& sm, int T, int hh, int kw, int lane,
                                         float& oa, float& ob, float& sum) {
  if (sm.slow[T & 1][hh])
    chain_tile<true, SUM>(sm, T, hh, kw, lane, oa, ob, sum);
  else
    chain_tile<false, SUM>(sm, T, hh, kw, lane, oa, ob, sum);
}

// Block = (KV head, chain, query-head pair): compute waves 0,1 own head 0 and
// 2,3 head 1, two adjacent value dims per thread. Wave 4 only moves data
// (global->LDS DMA), so no compute wave waits on memory counters, and waves
// 5 and 6 only turn head 0's and head 1's scores into exps, one tile ahead,
// so that work runs beside the value steps instead of before them. Waves 0
// and 3 also keep their head's sum (the SIMDs that host no exps wave). Per
// tile T: the producer waits until tiles up to T+1 are in LDS; barrier; the
// producer issues tile T+3 into the stage tile T-1 used; the exps waves form
// the exps of tile T+1; the compute waves run tile T.
constexpr int kChainThreads = 7 * 64;

__global__ __launch_bounds__(kChainThreads, 1) void k_attn_chain(AttnArgs a) {
  __shared__ ChainSmem sm;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const bool producer = wave == 4;
  const bool exps_wave = wave >= 5;
  const int hh = exps_wave ? wave - 5 : wave >> 1, kw = (wave & 1) * 64 + lane;  // dims 2kw, 2kw+1
  const bool sum_wave = wave == 0 || wave == 3;
  const int bx = blockIdx.x;
  const int hp = (bx >> 3) & 1, rest = (bx & 7) | ((bx >> 4) << 3);
  const int kvh = rest >> 6, c = rest & 63;
  const int pos = load_pos(a.st, a.pos_val);
  const int n = pos + 1;
  const int C = route_chains(n);
  if (c >= C) return;
  const int L = n > c ? (n - 1 - c) / C + 1 : 0;
  const int h0 = 4 * kvh + 2 * hp;
  float oa = 0.0f, ob = 0.0f, sum = 0.0f;
  float carry = kFiniteMin;  // exps waves: running max of their head
  if (L > 0) {
    const int nt = (L + kTile - 1) / kTile;
    const int sstride = score_stride(a.capacity);
    const uint16_t* vrow0 = a.vcache + ((size_t)kvh * a.capacity + c) * 256;
    const float* sc0 = a.scores + ((size_t)h0 * kAttnMaxChains + c) * sstride;
    if (producer) {
      for (int T = 0; T < kStages - 1 && T < nt; ++T) issue_tile(sm, vrow0, sc0, sstride, C, L, T, lane);
      // tile 0 complete; tiles 1 and 2 may stay pending (at most 63 operations
      // are ever outstanding, and loads complete in order)
      if (nt >= 3) wait_vm<63>(); else if (nt == 2) wait_vm<kTileOps>(); else wait_vm<0>();
    }
    // The producer keeps its DMA in flight across barriers (lds_barrier); the
    // other waves have no vector-memory operations outstanding and use
    // __syncthreads, whose waits the compiler tracks (an explicit wait that
    // leaves DMA pending makes it drain every LDS read instead).
    if (producer) lds_barrier(); else __syncthreads();
    // One loop per role, each with one barrier per tile.
    if (producer) {
      for (int T = 0; T < nt; ++T) {
        // tiles up to T+1 complete (V of T, scores of T+1); tile T+2 may pend
        if (T + 2 < nt) wait_vm<kTileOps>(); else wait_vm<0>();
        lds_barrier();
        if (T + kStages - 1 < nt) issue_tile(sm, vrow0, sc0, sstride, C, L, T + kStages - 1, lane);
      }
    } else if (exps_wave) {
      tile_exps(sm, 0, L, hh, lane, carry);
      for (int T = 0; T < nt; ++T) {
        __syncthreads();
        if (T + 1 < nt) tile_exps(sm, T + 1, L, hh, lane, carry);
      }
    } else if (sum_wave) {
      for (int T = 0; T < nt; ++T) {
        __syncthreads();
        run_tile<true>(sm, T, hh, kw, lane, oa, ob, sum);
      }
    } else {
      for (int T = 0; T < nt; ++T) {
        __syncthreads();
        run_tile<false>(sm, T, hh, kw, lane, oa, ob, sum);
      }
    }
  }
  if (producer) return;
  float* ml = a.part_ml + ((size_t)(h0 + hh) * kAttnMaxChains + c) * 2;
  if (exps_wave) {
    if (lane == 0) ml[0] = carry;
    return;
  }
  float* po = a.part_o + ((size_t)(h0 + hh) * kAttnMaxChains + c) * 256 + 2 * kw;
  *reinterpret_cast<float2*>(po) = make_float2(oa, ob);
  if (sum_wave && lane == 0) ml[1] = sum;
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
  return (size_t)kQHeads * kAttnMaxChains * (256 + 2 + score_stride(capacity)) * sizeof(float);
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
  hipLaunchKernelGGL(k_attn_chain, dim3(kKvHeads * kAttnMaxChains * 2), dim3(kChainThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_attn_merge(const AttnArgs& a, hipStream_t s) {
  if (!attn_ok(a)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_merge, dim3(kQHeads, 4), dim3(64), 0, s, a);
  return hipGetLastError();
}

}  // namespace es
