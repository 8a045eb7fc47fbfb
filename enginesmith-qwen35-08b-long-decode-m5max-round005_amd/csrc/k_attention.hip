// GQA decode attention on gfx950 (8 query heads, 2 KV heads, head dim 256,
// one query token), computing the reference's own two routes
// (model.rs:327-347) in a fixed fp32 order:
//   length < 1024: 32 position chains (chain c takes positions c, c+32, ...),
//     combined in fp32 (sdpa_vector, attention_decode.metal:51-213);
//   length >= 1024: 64 chains whose unnormalised outputs are rounded to bf16,
//     then merged and gated (sdpa_vector_2pass_1 + attn_decode_split2_gate,
//     attention_decode.metal:215-431, 830-891).
//
// k_attn_fused, 256 blocks x 768 threads: block = (KV head, chain, query-head
//   pair). The prologue fuses attn_prepare_qkv_decode (attention.metal:262-313:
//   q/k RMSNorm with bf16 normalised value and bf16 gain product, RoPE on dims
//   0..63 with pairs (i, i+32)); the blocks of the chain that holds the new
//   position form its K/V rows, write them to the cache (query-head pair 0)
//   and use them in place of the rows they stream. Two data-moving waves
//   stage the chain's K and V rows in LDS by 16-byte global->LDS DMA, 32-step
//   tiles, four deep. Four waves score each K tile for both heads
//   (8 lanes per position, lane m holds dims 8m+64i .. +7 (i = 0..3), one fma
//   chain per 8 dims, (p[m]+p[m+8])+(p[m+16]+p[m+24]) in the lane and a DPP
//   tree over the 8 lanes); two waves turn the scores into running max,
//   factor and exp score one tile later (max scan by DPP, exp by the shared
//   series), which reach the chain lanes by DPP row broadcast; four waves
//   run the chain steps two tiles after the scores, per step
//   o = fma(e, v, o*factor) and sum = sum*factor + e; when every factor of a
//   tile is exactly 1 the products by 1 are skipped, which changes no bit.
//   K and V are each read from HBM once; the two blocks of a (KV head, chain)
//   sit on the same XCD (block ids b and b+8) so the second read of each row
//   is an L2 hit.
// k_attn_merge, grid (8 heads, 4 quarters) x 64: chain combination of either
//   route, then gated = bf16(bf16(o) * sigmoid_bf(gate)) (attention.metal:133-151).
#include "es_kernels.hpp"

namespace es {
namespace {

constexpr float kFiniteMin = -3.40282346638528859812e38f;

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

__device__ __forceinline__ int route_chains(int n) { return n < kAttnRouteSplit ? 32 : 64; }

// ---- fused scores + per-chain online softmax ----

constexpr int kTile = 32;     // chain steps per tile
constexpr int kStages = 4;    // K and V tiles in LDS, each ring four deep
constexpr int kTileOps = 16;  // DMA operations per tile and ring (2 rows each)

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

struct __attribute__((aligned(16))) FusedSmem {
  uint16_t k[kStages][kTile][256];  // K rows of a tile, as loaded
  uint16_t v[kStages][kTile][256];  // V rows of a tile, as loaded
  float s[2][2][kTile];             // [buffer][head][step] scores
  float e[2][2][kTile];             // exp scores
  float f[2][2][kTile];             // factors
  int slow[2][2];                   // some factor of the tile differs from 1
  float qs[2][256];                 // roped q x 1/16 of both heads
  u32x4 knew[32];                   // new K row (roped, bf16)
  u32x4 vnew[32];                   // new V row
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

// Wait until tile t has landed when `later` (0..2) tiles of the same ring
// were issued after it.
__device__ __forceinline__ void wait_tiles(int later) {
  if (later >= 2) wait_vm<2 * kTileOps>();
  else if (later == 1) wait_vm<kTileOps>();
  else wait_vm<0>();
}

// Issue tile t of one ring (K or V rows of the chain) from a producer wave:
// 32 rows as 16 DMA of 1 KB (lanes 0..31 one row, 32..63 the next). Rows
// past the chain's end re-read its last row (in bounds; their scores are
// masked and their exp scores are 0). The reads are non-temporal: the KV
// stream is far larger than the on-package cache and would otherwise evict
// the weights the small kernels read again next step.
__device__ __forceinline__ void issue_rows(uint16_t (*ring)[kTile][256], const uint16_t* row0, int C,
                                           int L, int t, int lane) {
  uint16_t(*dst)[256] = ring[t % kStages];
#pragma unroll 4
  for (int x = 0; x < kTile / 2; ++x) {
    const int r = 2 * x;
    const int j = min(t * kTile + r + (lane >> 5), L - 1);
    const uint16_t* g = row0 + (size_t)j * C * 256 + (lane & 31) * 8;
    __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)&dst[r][0], 16, 0, kLoadNonTemporal);
  }
}

// Overwrite row i of a staged tile with the row computed in this launch
// (the cache row may still hold the old value when the DMA read it).
__device__ __forceinline__ void patch_row(uint16_t* row, const u32x4* src, int lane) {
  if (lane < 32) reinterpret_cast<u32x4*>(row)[lane] = src[lane];
}

// Scores of tile t for both heads of the block: 8 lanes per position, lane m
// holds dims 8m+64x .. +7 (x = 0..3) of the K row; one fma chain per 8 dims,
// (p[m]+p[m+8])+(p[m+16]+p[m+24]) in the lane and a DPP tree over the 8
// lanes. The four compute waves cover the tile's 32 positions.
__device__ __forceinline__ void tile_scores(FusedSmem& sm, int t, int pidx, int m,
                                            const float (&q)[2][4][8]) {
  const u32x4* row = reinterpret_cast<const u32x4*>(&sm.k[t % kStages][pidx][0]);
  u32x4 kc[4];
#pragma unroll
  for (int x = 0; x < 4; ++x) kc[x] = row[m + 8 * x];
  float s[2];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const float p0 = chunk_dot(q[hh][0], kc[0]);
    const float p1 = chunk_dot(q[hh][1], kc[1]);
    const float p2 = chunk_dot(q[hh][2], kc[2]);
    const float p3 = chunk_dot(q[hh][3], kc[3]);
    s[hh] = tree8((p0 + p1) + (p2 + p3));
  }
  if (m < 2) sm.s[t & 1][m][pidx] = m == 0 ? s[0] : s[1];
}

// Exp scores and factors of tile t for one head from its scores (lanes 0..31
// hold the tile's steps; lanes past the tile or the chain read -inf).
__device__ __forceinline__ void tile_exps(FusedSmem& sm, int t, int L, int head, int lane,
                                          float& carry) {
  const float ninf = -__builtin_inff();
  const float s = lane < kTile && t * kTile + lane < L ? sm.s[t & 1][head][lane] : ninf;
  const float mt = fmaxf(carry, wave_max_scan(s));
  const float pv = dpp_src<0x138, 0xf>(mt, carry);  // wave_shr:1, lane 0 <- carry
  const float f = es_exp(pv - mt), e = es_exp(s - mt);
  if (lane < kTile) {
    sm.e[t & 1][head][lane] = e;
    sm.f[t & 1][head][lane] = f;
  }
  sm.slow[t & 1][head] = __any(f != 1.0f);  // wave-uniform, stored by every lane
  carry = readlane63(mt);
}

// Exp scores and factors reach the compute waves through DPP: each lane
// holds e[16r + (lane & 15)] for r = 0, 1 (one 4-byte LDS read per r), and
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

// Groups G .. 3 of a tile: compute group G, then issue the loads of group
// G + AHEAD into the slot it frees. LDS reads complete in order and at most
// 15 may be outstanding (the counter's width), so a fast tile keeps three
// groups in flight (plus one read of exp scores) and a slow tile, which also
// reads factors, two.
template <int G, bool SLOW, bool SUM>
__device__ __forceinline__ void chain_groups(const uint32_t* vw, int kw, const float* er,
                                             const float* fr, uint32_t (&w)[4][8], float& oa,
                                             float& ob, float& sum) {
  if constexpr (G < kTile / 8) {
    constexpr int ahead = SLOW ? 2 : 3;
    chain_group<G, SLOW, SUM>(w[G % 4], er[G / 2], fr[G / 2], oa, ob, sum);
    issue_fence();
    if constexpr (G + ahead < kTile / 8) {
      load_group(vw, kw, G + ahead, w[(G + ahead) % 4]);
      issue_fence();
    }
    chain_groups<G + 1, SLOW, SUM>(vw, kw, er, fr, w, oa, ob, sum);
  }
}

// The tile's steps for the two adjacent dims owned by this thread for one
// head; SUM waves also keep the head's sum. Steps past the chain's end have
// e = 0 and f = 1 and change nothing (o is never -0, V rows are finite).
template <bool SLOW, bool SUM>
__device__ __forceinline__ void chain_tile(const FusedSmem& sm, int t, int hh, int kw, int lane,
                                           float& oa, float& ob, float& sum) {
  const uint32_t* vw = reinterpret_cast<const uint32_t*>(&sm.v[t % kStages][0][0]);
  const float* ep = sm.e[t & 1][hh] + (lane & 15);
  const float* fp = sm.f[t & 1][hh] + (lane & 15);
  float er[2], fr[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
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
__device__ __forceinline__ void run_tile(const FusedSmem& sm, int t, int hh, int kw, int lane,
                                         float& oa, float& ob, float& sum) {
  if (sm.slow[t & 1][hh])
    chain_tile<true, SUM>(sm, t, hh, kw, lane, oa, ob, sum);
  else
    chain_tile<false, SUM>(sm, t, hh, kw, lane, oa, ob, sum);
}

// Block = (KV head, chain, query-head pair), 12 waves, three per SIMD. Waves
// 0..3 run the chain for head (wave & 1), two adjacent value dims per thread
// (waves 0 and 1 also keep their head's sum); waves 4..7 score the tiles, 8
// lanes per position; wave 8 streams the chain's K rows and wave 9 its V rows
// into LDS by global->LDS DMA; waves 10 and 11 turn head 0's and head 1's
// scores into exps. Each SIMD hosts one chain wave and one scoring wave, so
// one's LDS latency is covered by the other's arithmetic. Iteration I (one
// barrier each): scores of tile I, exps of tile I-1, chain steps of tile
// I-2; K tile I+3 and V tile I+1 are issued into the stages freed by tiles
// I-1 and I-3.
constexpr int kFusedThreads = 12 * 64;

__global__ __launch_bounds__(kFusedThreads, 1) void k_attn_fused(AttnArgs a) {
  __shared__ FusedSmem sm;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int bx = blockIdx.x;
  const int hp = (bx >> 3) & 1, rest = (bx & 7) | ((bx >> 4) << 3);
  const int kvh = rest >> 6, c = rest & 63;
  const int pos = load_pos(a.st, a.pos_val);
  const int n = pos + 1;
  const int C = route_chains(n);
  if (c >= C) return;
  const int L = n > c ? (n - 1 - c) / C + 1 : 0;
  const int nt = (L + kTile - 1) / kTile;
  const int h0 = 4 * kvh + 2 * hp;
  const bool holder = pos % C == c;  // this chain's last step is the new position
  const int jpos = pos / C, tpos = jpos / kTile, ipos = jpos % kTile;
  const uint16_t* krow0 = a.kcache + ((size_t)kvh * a.capacity + c) * 256;
  const uint16_t* vrow0 = a.vcache + ((size_t)kvh * a.capacity + c) * 256;

  // ---- prologue: producers start streaming; the others form q (and, in
  // the holder blocks, the new K/V rows) ----
  if (wave == 8) {
    for (int tt = 0; tt < 3 && tt < nt; ++tt) issue_rows(sm.k, krow0, C, L, tt, lane);
  } else if (wave == 9) {
    if (nt > 0) issue_rows(sm.v, vrow0, C, L, 0, lane);
  } else if (wave < 4) {
    // One barrier: RoPE takes the partner dims (d ^ 32, in lane ^ 8) by DPP,
    // so q and the new K row go to LDS straight after the norm.
    uint2 xv, gv;
    float inv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (wave < 2) {
      xv = *reinterpret_cast<const uint2*>(a.q_proj + (h0 + wave) * 512 + lane * 4);
      gv = *reinterpret_cast<const uint2*>(a.q_gain + lane * 4);
    } else {
      xv = *reinterpret_cast<const uint2*>((wave == 2 ? a.k_proj : a.v_proj) + kvh * 256 + lane * 4);
      gv = *reinterpret_cast<const uint2*>(a.k_gain + lane * 4);
    }
    if (wave < 3) {
#pragma unroll
      for (int x = 0; x < 4; ++x) inv[x] = a.inv_freq[((lane * 4) & 31) + x];
    }
    issue_fence();
    if (wave < 3) {
      float o4[4], p4[4], r[4];
      head_norm4(xv, gv, o4);
#pragma unroll
      for (int x = 0; x < 4; ++x) p4[x] = dpp_row_ror8(o4[x]);
#pragma unroll
      for (int x = 0; x < 4; ++x) r[x] = rope_at(o4[x], p4[x], lane * 4 + x, pos, inv[x]);
      if (wave < 2) {
        if (a.query_out && c == 0) {
          uint16_t* qo = a.query_out + (h0 + wave) * 256 + lane * 4;
          *reinterpret_cast<uint2*>(qo) = make_uint2(pack_bf2(r[0], r[1]), pack_bf2(r[2], r[3]));
        }
#pragma unroll
        for (int x = 0; x < 4; ++x) sm.qs[wave][lane * 4 + x] = r[x] * 0.0625f;
      } else {
        const uint2 kp = make_uint2(pack_bf2(r[0], r[1]), pack_bf2(r[2], r[3]));
        reinterpret_cast<uint2*>(sm.knew)[lane] = kp;
        if (holder && hp == 0)
          *reinterpret_cast<uint2*>(a.kcache + ((size_t)kvh * a.capacity + pos) * 256 + lane * 4) = kp;
      }
    } else {
      reinterpret_cast<uint2*>(sm.vnew)[lane] = xv;
      if (holder && hp == 0)
        *reinterpret_cast<uint2*>(a.vcache + ((size_t)kvh * a.capacity + pos) * 256 + lane * 4) = xv;
    }
  }
  if (wave == 8 || wave == 9) lds_barrier(); else __syncthreads();

  float oa = 0.0f, ob = 0.0f, sum = 0.0f;
  float carry = kFiniteMin;  // exps waves: running max of their head
  // One loop per role, each with one barrier per iteration. The producers
  // keep DMA in flight across barriers (lds_barrier); the other waves have no
  // vector-memory operations outstanding and use __syncthreads, whose waits
  // the compiler tracks.
  if (wave == 8) {
    for (int I = 0; I < nt + 2; ++I) {
      if (I < nt) {
        wait_tiles(min(2, nt - 1 - I));  // K tile I landed
        if (holder && I == tpos) patch_row(&sm.k[I % kStages][ipos][0], sm.knew, lane);
      }
      lds_barrier();
      if (I + 3 < nt) issue_rows(sm.k, krow0, C, L, I + 3, lane);
    }
  } else if (wave == 9) {
    for (int I = 0; I < nt + 2; ++I) {
      if (I >= 2) {
        wait_tiles(min(2, nt - 1 - (I - 2)));  // V tile I-2 landed
        if (holder && I - 2 == tpos) patch_row(&sm.v[(I - 2) % kStages][ipos][0], sm.vnew, lane);
      }
      lds_barrier();
      if (I + 1 < nt) issue_rows(sm.v, vrow0, C, L, I + 1, lane);
    }
  } else if (wave >= 10) {
    const int head = wave - 10;
    for (int I = 0; I < nt + 2; ++I) {
      __syncthreads();
      if (I >= 1 && I <= nt) tile_exps(sm, I - 1, L, head, lane, carry);
    }
  } else if (wave >= 4) {
    const int pidx = (wave - 4) * 8 + (lane >> 3), m = lane & 7;
    float q[2][4][8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int j = 0; j < 8; ++j) q[h][x][j] = sm.qs[h][64 * x + 8 * m + j];
    for (int I = 0; I < nt + 2; ++I) {
      __syncthreads();
      if (I < nt) tile_scores(sm, I, pidx, m, q);
    }
  } else {
    const int hh = wave & 1, kw = (wave >> 1) * 64 + lane;  // dims 2kw, 2kw+1
    const bool sum_wave = wave < 2;
    for (int I = 0; I < nt + 2; ++I) {
      __syncthreads();
      if (I >= 2) {
        if (sum_wave) run_tile<true>(sm, I - 2, hh, kw, lane, oa, ob, sum);
        else run_tile<false>(sm, I - 2, hh, kw, lane, oa, ob, sum);
      }
    }
    float* po = a.part_o + ((size_t)(h0 + hh) * kAttnMaxChains + c) * 256 + 2 * kw;
    *reinterpret_cast<float2*>(po) = make_float2(oa, ob);
    if (sum_wave && lane == 0) a.part_ml[((size_t)(h0 + hh) * kAttnMaxChains + c) * 2 + 1] = sum;
    return;
  }
  if (wave >= 10 && lane == 0) a.part_ml[((size_t)(h0 + wave - 10) * kAttnMaxChains + c) * 2] = carry;
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

// Chain factors of head h for the merge, by one 64-lane wave: fac[l] =
// exp(max_l - max) and *total = the weighted sum of the chain sums
// (attention_decode.metal:858-862 for the long route).
// The (max, sum) pair of chain `lane` (lane & 31 on the short route).
__device__ __forceinline__ float2 load_chain_ml(const AttnArgs& a, int h, int lane, bool two_pass) {
  const float* ml = a.part_ml + (size_t)h * kAttnMaxChains * 2;
  return reinterpret_cast<const float2*>(ml)[two_pass ? lane : (lane & 31)];
}

__device__ __forceinline__ void merge_factors(float2 mlv, int lane, bool two_pass, float* fac,
                                              float* total) {
  if (two_pass) {
    const float mx = mlv.x;
    const float F = es_exp(mx - wave_max(mx));
    fac[lane] = F;
    // lane l < 32: (0 + F_l s_l) + F_{l+32} s_{l+32}, then pairwise over lanes
    const float prod = F * mlv.y;
    const float hi = rows_xor32(prod).y;  // lane l < 32: prod of lane l + 32
    float s = 0.0f;
    s = s + prod;
    s = s + hi;
    s = tree32(s);
    if (lane == 0) *total = s;
  } else {
    const float mx = lane < 32 ? mlv.x : kFiniteMin;
    const float F = es_exp(mx - wave_max(mx));
    if (lane < 32) fac[lane] = F;
    const float s = tree32(mlv.y * F);
    if (lane == 0) *total = s;
  }
}

// Merged, normalised and gated value of dim d of head h: bf16(bf16(o) *
// sigmoid_bf(gate)) with o = (sum of factor-weighted chain outputs) / total;
// v holds the 64 chain outputs of the dim (loaded by the caller).
// gate_raw: bf16 gate of the dim (q_proj[h*512 + 256 + d]).
__device__ __forceinline__ uint32_t merge_dim(uint32_t gate_raw, bool two_pass, const float* fac,
                                              float sum, float* v) {
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
  const float gate = sigmoid_bf(bf2f(gate_raw));
  return f2bf(attention * gate);
}

__device__ __forceinline__ void load_chain_outputs(const AttnArgs& a, int h, int d, bool two_pass,
                                                   float* v) {
  const float* po = a.part_o + (size_t)h * kAttnMaxChains * 256 + d;
#pragma unroll
  for (int c = 0; c < 32; ++c) v[c] = po[(size_t)c * 256];
  if (two_pass) {
#pragma unroll
    for (int c = 32; c < 64; ++c) v[c] = po[(size_t)c * 256];
  }
}

__global__ __launch_bounds__(64) void k_attn_merge(AttnArgs a) {
  __shared__ float fac[kAttnMaxChains];
  __shared__ float total;
  const int lane = threadIdx.x, h = blockIdx.x;
  const int d = blockIdx.y * 64 + lane;
  const int pos = load_pos(a.st, a.pos_val);
  const bool two_pass = pos + 1 >= kAttnRouteSplit;
  // (max, sum) pairs, chain outputs and the gate in flight together; the
  // factors form as soon as the first arrive.
  const float2 mlv = load_chain_ml(a, h, lane, two_pass);
  float v[kAttnMaxChains];
  load_chain_outputs(a, h, d, two_pass, v);
  const uint32_t gate_raw = a.q_proj[h * 512 + 256 + d];
  issue_fence();
  merge_factors(mlv, lane, two_pass, fac, &total);
  __syncthreads();
  a.gated[h * 256 + d] = (uint16_t)merge_dim(gate_raw, two_pass, fac, total, v);
}

// Engine path: merge + gate of head h (every one of the 32 blocks of the head
// forms all 256 dims; more blocks with fewer rows each finish sooner than 8
// blocks of 128 rows) and the head's share of o_proj for output rows
// 32*rg .. +31: per row the eight 32-column slice partials combined by
// tree8. The 64-slice tree of a K=2048 row pairs adjacent slices first, so the
// row's full sum is the pairwise tree8 of the 8 head partials, formed by the
// next launch, bit for bit.
constexpr int kMergeRows = 32;  // o_proj rows per block: 8 lanes per row

__global__ __launch_bounds__(256) void k_attn_merge_out(AttnArgs a, Q4 o, const uint32_t* o_sb, float* part) {
  __shared__ float fac[kAttnMaxChains];
  __shared__ float total;
  __shared__ float gx[256 + 8];  // gated output, slice s at gx[33 s ..]
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int h = blockIdx.x, rg = blockIdx.y;  // a head's blocks share an XCD
  const int sl = t & 7, gs = 8 * h + sl;  // K slice of this lane
  const int pos = load_pos(a.st, a.pos_val);
  const bool two_pass = pos + 1 >= kAttnRouteSplit;
  // Loads in the order they are needed (they complete in issue order): the
  // (max, sum) pairs, the chain outputs and the gate, then the o_proj slice.
  float2 mlv = make_float2(0.0f, 0.0f);
  if (wave == 0) mlv = load_chain_ml(a, h, lane, two_pass);
  float v[kAttnMaxChains];
  load_chain_outputs(a, h, t, two_pass, v);
  const uint32_t gate_raw = a.q_proj[h * 512 + 256 + t];
  issue_fence();
  const size_t row = (size_t)kMergeRows * rg + (t >> 3);
  const u32x4 oc = *reinterpret_cast<const u32x4*>(o.w + row * 256 + gs * 4);
  // the head's four group words of the row, contiguous (launch_pack_out_pairs)
  const uint32_t osb = o_sb[((size_t)h * 1024 + row) * 4 + sl / 2];
  issue_fence();
  if (wave == 0) merge_factors(mlv, lane, two_pass, fac, &total);
  __syncthreads();
  gx[t + (t >> 5)] = bf2f(merge_dim(gate_raw, two_pass, fac, total, v));
  __syncthreads();
  float xv[32], xr[32];
#pragma unroll
  for (int q = 0; q < 32; ++q) xv[q] = gx[sl * 33 + q];
  const float xs = prep_slice(xv, xr);
  const float pp = tree8(q4_slice_sb(oc, osb, xr, xs));
  if (sl == 0) part[(size_t)h * 1024 + row] = pp;
}

bool attn_ok(const AttnArgs& a) {
  return a.q_proj && a.k_proj && a.v_proj && a.q_gain && a.k_gain && a.kcache && a.vcache &&
         a.inv_freq && a.part_o && a.part_ml && a.gated && a.blocks >= 1 &&
         a.blocks <= 1024 && a.capacity > 0 &&
         (a.st || (a.pos_val >= 0 && a.pos_val < a.capacity));
}

}  // namespace

size_t attn_scratch_bytes(int capacity) {
  (void)capacity;  // the chain states do not grow with the cache
  return (size_t)kQHeads * kAttnMaxChains * (256 + 2) * sizeof(float);
}

void attn_bind_scratch(AttnArgs& a, void* scratch) {
  a.part_o = static_cast<float*>(scratch);
  a.part_ml = a.part_o + (size_t)kQHeads * kAttnMaxChains * 256;
}

hipError_t launch_attn_fused(const AttnArgs& a, hipStream_t s) {
  if (!attn_ok(a)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_fused, dim3(kKvHeads * kAttnMaxChains * 2), dim3(kFusedThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_attn_merge_out(const AttnArgs& a, const Q4& o, const uint32_t* o_sb, float* part,
                                 hipStream_t s) {
  if (!attn_ok(a) || !o.w || !o_sb || o.n != kHidden || o.k != 2048 || !part) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_merge_out, dim3(kQHeads, kHidden / kMergeRows), dim3(256), 0, s, a, o, o_sb, part);
  return hipGetLastError();
}

hipError_t launch_attn_merge(const AttnArgs& a, hipStream_t s) {
  if (!attn_ok(a)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_merge, dim3(kQHeads, 4), dim3(64), 0, s, a);
  return hipGetLastError();
}

}  // namespace es
