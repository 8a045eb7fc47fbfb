// Decode kernels whose blocks cooperate within one XCD.
//
// MI355X deals the workgroups of a launch to its 8 XCDs in turn, starting
// where the previous launch stopped, so each XCD receives 32 blocks of a
// 256-block launch and the blocks of one XCD have distinct b >> 3. A block
// takes its XCD from the XCC_ID hardware register and its rank within the XCD
// from b >> 3. The 32 blocks of an XCD share its L2 and exchange data through
// it (tagged words, below) at the cost of one store and one load, where any
// exchange between XCDs costs a kernel boundary. The engine uses these kernels only
// after a start-up probe has seen that dealing. Waits are bounded and fail
// fast: a wait that exceeds kSpinLimit polls (as it would if two blocks of one
// XCD shared a rank) sets an error word; every 64th poll of any wait reads
// that word and gives up once it is set, and a launch that starts with the
// word set makes no wait at all. The kernels index nothing by exchanged
// values, so a wait that gave up leaves wrong numbers but no stray access; the
// engine checks the word after each batch of steps, reports the error, and
// clears the word, the exchange counts and the exchange words.
//
// k_mlp_xcd: the MLP of a layer in one launch. It replaces the post-mixer
// residual + post RMSNorm + gate/up + SwiGLU launch and the down-projection
// launch. The K=3584 down row's canonical sum is tree64 over 64 lanes whose
// leaf l holds slices l and l + 64 (l < 48) or slice l; its first three levels
// are the sums of the eight octets of leaves, and the rest is the pairwise sum
// of the eight octet sums in index order. XCD x computes the activation
// elements octet x needs (slices 8x..8x+7 and, for x < 6, 8x+64..8x+71: 512
// or 256 elements), exchanges them within the XCD, and writes octet x's sum of
// every output row. The next launch adds the eight octet sums pairwise and the
// residual, so the layer's output is bit for bit the two-launch result.
#include "es_kernels.hpp"

namespace es {
namespace {

constexpr int kGroupBlocks = 32;          // blocks per XCD in a 256-block launch
constexpr int kSpinLimit = 1 << 16;       // polls before a wait gives up (tens of ms)

__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 15u;
}

// After a failed poll n of a wait: true when the wait is to stop. Every 64th
// poll checks the limit (setting the error word when it has run out) and reads
// the error word that another wait may have set (an agent-scope load: the
// word is set by atomics from any XCD).
__device__ __forceinline__ bool wait_gives_up(int n, uint32_t* err) {
  if ((n & 63) != 63) return false;
  if (n >= kSpinLimit) {
    atomicOr(err, 2u);
    return true;
  }
  return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}

// Exchanges within an XCD are tagged words: each published word holds a bf16
// value in its low half and the exchange's tag in its high half, written whole
// by one aligned 32-bit store (the L1 writes through to the XCD's L2), so a
// word that carries the tag holds this exchange's value, and a reader polls
// the data itself with loads that miss the L1 (sc1). That is one memory round
// trip after the last write, where a barrier on flags takes four (the
// writer's store acknowledgement, its flag store, the flag poll, the data
// load). The tag is the low 16 bits of the block's exchange count: flags[rank]
// holds the count as the block left its previous launch, and every block of an
// XCD makes the same exchanges, so the counts agree at each launch start; a
// launch with E exchanges uses count + 1 .. count + E and stores count + E.
// Consecutive writes of a word are at most a few exchanges apart, so they
// carry different tags (the words and counts start at 0, the first tag is 1).
//
// xcd_gather: wave 0 reads the `count` words (8 per lane) until every one
// carries `tag`, and writes their values to lds (slice k of 32 at lds[36k ..]);
// the block then syncs.
__device__ __forceinline__ void xcd_gather(const uint32_t* words, int count, uint32_t tag, float* lds,
                                           uint32_t* err, bool failed) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const bool live = lane * 8 < count;
    const uint32_t* p = words + (live ? lane * 8 : 0);
    u32x4 w0, w1;
    for (int n = 0;; ++n) {
      asm volatile(
          "global_load_dwordx4 %0, %2, off sc1\n\t"
          "global_load_dwordx4 %1, %2, off offset:16 sc1\n\t"
          "s_waitcnt vmcnt(0)"
          : "=&v"(w0), "=&v"(w1)
          : "v"(p)
          : "memory");
      bool ok = true;
#pragma unroll
      for (int i = 0; i < 4; ++i) ok = ok && (w0[i] >> 16) == tag && (w1[i] >> 16) == tag;
      if (__all(ok || !live) || failed || wait_gives_up(n, err)) break;
    }
    if (live) {
      float4* d = reinterpret_cast<float4*>(lds + (lane >> 2) * 36 + (lane & 3) * 8);
      d[0] = make_float4(bf_lo(w0[0]), bf_lo(w0[1]), bf_lo(w0[2]), bf_lo(w0[3]));
      d[1] = make_float4(bf_lo(w1[0]), bf_lo(w1[1]), bf_lo(w1[2]), bf_lo(w1[3]));
    }
  }
  __syncthreads();
}

template <int N>
__device__ __forceinline__ float pair_sum(const float* v) {
  if constexpr (N == 1) {
    return v[0];
  } else {
    return pair_sum<N / 2>(v) + pair_sum<N / 2>(v + N / 2);
  }
}

// Activation elements of XCD x's octet, in exchange order: j < 256 is element
// 256x + j, j >= 256 (x < 6) element 2048 + 256x + (j - 256).
__device__ __forceinline__ int octet_act(int x, int j) { return j < 256 ? 256 * x + j : 2048 + 256 * x + (j - 256); }

template <int NPART>
__global__ __launch_bounds__(256) void k_mlp_xcd(MlpXcdArgs a) {
  __shared__ float hs[kNormLds];
  __shared__ float norm_lds[kNormLds];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, half = lane >> 5, sl = lane & 31;
  const int x = (int)xcc_id() & 7, rank = blockIdx.x >> 3;
  const int nact = x < 6 ? 16 : 8;  // activation elements of this block
  uint32_t* flags = a.flags + x * kGroupBlocks;
  // every pointer argument in scalar registers at once (one wait)
  asm volatile("" :: "s"(a.gate.w), "s"(a.up.w), "s"(a.gu_sb), "s"(a.down.w), "s"(a.down_sb), "s"(a.h_old),
               "s"(a.part), "s"(a.h_mid), "s"(a.gain), "s"(a.dpart), "s"(a.xact), "s"(a.flags), "s"(a.err));

  // ---- loads: residual, gain and mixer partials; the exchange count;
  // gate/up weights; the down weights of phase 2
  const uint2 ho = reinterpret_cast<const uint2*>(a.h_old)[t];
  const uint2 g4 = reinterpret_cast<const uint2*>(a.gain)[t];
  float4 pv[NPART];
#pragma unroll
  for (int k = 0; k < NPART; ++k) pv[k] = reinterpret_cast<const float4*>(a.part + k * kHidden)[t];
  // this block's exchange count as it left the previous launch; the error
  // word (set: make no wait), first used at the exchange
  const uint32_t own = flags[rank];
  uint32_t err_raw = *a.err;
  issue_fence();
  u32x4 cg[2], cu[2];
  uint32_t gsb[2], usb[2];
  int er[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int j = wave * 4 + 2 * p + half;  // local row in the block
    const int e = j < nact ? octet_act(x, rank * nact + j) : 0;
    er[p] = j < nact ? e : -1;
    cg[p] = *reinterpret_cast<const u32x4*>(a.gate.w + (size_t)e * 128 + sl * 4);
    cu[p] = *reinterpret_cast<const u32x4*>(a.up.w + (size_t)e * 128 + sl * 4);
    const uint2 gu = a.gu_sb[(size_t)e * 16 + sl / 2];
    gsb[p] = gu.x;
    usb[p] = gu.y;
  }
  // phase 2: down rows 32 rank .. +31; x < 6: 16 lanes per row (lane L holds
  // slice 8x+L, or 8x+64+L-8 for L >= 8), two passes of 16 rows; x >= 6: 8
  // lanes per row (slice 8x+L), one pass of 32 rows
  const int wide = x < 6;
  const int L = wide ? (t & 15) : (t & 7);
  const int dslice = wide ? (L < 8 ? 8 * x + L : 8 * x + 64 + (L - 8)) : 8 * x + L;
  const int dword = L < 8 ? L / 2 : 4 + (L - 8) / 2;  // its group's word in the octet's row
  u32x4 dc[2];
  uint32_t dsb[2];
  int drow[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int row = wide ? rank * 32 + p * 16 + (t >> 4) : rank * 32 + (t >> 3);
    drow[p] = row;
    dc[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.down.w + (size_t)row * 448 + dslice * 4));
    dsb[p] = __builtin_nontemporal_load(a.down_sb + ((size_t)x * 1024 + row) * 8 + dword);
  }
  issue_fence();

  // ---- phase 1: h = bf16(h_old + bf16(pairwise sum of the mixer partials)),
  // post RMSNorm, this block's gate/up rows and SwiGLU (k_norm_gate_up_parts)
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
  if (blockIdx.x == 0) reinterpret_cast<uint2*>(a.h_mid)[t] = x4;
  *reinterpret_cast<float4*>(hs + (t >> 3) * 36 + (t & 7) * 4) = make_float4(hn[0], hn[1], hn[2], hn[3]);
  __syncthreads();
  float xv[32];
  {
    const float4* rp = reinterpret_cast<const float4*>(hs + sl * 36);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 q = rp[i];
      xv[4 * i] = q.x; xv[4 * i + 1] = q.y; xv[4 * i + 2] = q.z; xv[4 * i + 3] = q.w;
    }
  }
  float xn[32];
  norm_block_1024(xv, x4, g4, norm_lds, xn);
  float xr[32];
  float xs = prep_slice(xn, xr);
  uint32_t* xact = a.xact + x * 512;
  const uint32_t tag = (own + 1u) & 0xffffu;
  float gv[2], uv[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    gv[p] = tree32(q4_slice_sb(cg[p], gsb[p], xr, xs));
    uv[p] = tree32(q4_slice_sb(cu[p], usb[p], xr, xs));
  }
  // lane p < 2 of each half-wave forms element p's SwiGLU (every lane holds
  // both sums)
  if (sl < 2 && (sl == 0 ? er[0] : er[1]) >= 0) {
    const float gb = rbf(sl == 0 ? gv[0] : gv[1]), ub = rbf(sl == 0 ? uv[0] : uv[1]);
    const float silu = rbf(gb * sigmoid_bf(gb));
    xact[rank * nact + wave * 4 + 2 * sl + half] = f2bf(silu * ub) | tag << 16;
  }

  // ---- exchange the XCD's activation elements (hs is free again: the
  // norm's barrier followed its last read)
  if (t == 0) flags[rank] = own + 1u;
  // the error word is read here, not at entry: a uniform value formed from a
  // load right after it would wait for every input load before the weights
  // are issued
  asm volatile("" : "+v"(err_raw));
  xcd_gather(xact, wide ? 512 : 256, tag, hs, a.err, err_raw != 0u);

  // ---- phase 2: octet x of every down row of this block
  // lane L's slice: elements 32L .. 32L+31 of the exchange
  {
    const float4* rp = reinterpret_cast<const float4*>(hs + L * 36);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 q = rp[i];
      xv[4 * i] = q.x; xv[4 * i + 1] = q.y; xv[4 * i + 2] = q.z; xv[4 * i + 3] = q.w;
    }
  }
  xs = prep_slice(xv, xr);
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    if (!wide && p == 1) break;
    float v = q4_slice_sb(dc[p], dsb[p], xr, xs);
    if (wide) v = v + dpp_row_ror8(v);  // leaf: slices 8x+L and 8x+64+L
    v = tree4(v);
    v = v + dpp_half_mirror(v);         // the octet's tree over its 8 leaves
    if (L == 0) a.dpart[x * kHidden + drow[p]] = v;
  }
}

// Two tagged exchange words (xcd_gather's format) read by each lane from the
// XCD's L2 until the first carries tag0 and the second tag1; returns their
// bf16 values.
__device__ __forceinline__ uint2 xcd_poll2(const uint32_t* p0, uint32_t tag0, const uint32_t* p1, uint32_t tag1,
                                           uint32_t* err, bool failed) {
  uint32_t a, b;
  for (int n = 0;; ++n) {
    asm volatile(
        "global_load_dword %0, %2, off sc1\n\t"
        "global_load_dword %1, %3, off sc1\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(a), "=&v"(b)
        : "v"(p0), "v"(p1)
        : "memory");
    if (__all((a >> 16) == tag0 && (b >> 16) == tag1) || failed || wait_gives_up(n, err)) break;
  }
  return make_uint2(a & 0xffffu, b & 0xffffu);
}

// The same for three words with one tag.
__device__ __forceinline__ uint3 xcd_poll3(const uint32_t* p0, const uint32_t* p1, const uint32_t* p2, uint32_t tag,
                                           uint32_t* err, bool failed) {
  uint32_t a, b, c;
  for (int n = 0;; ++n) {
    asm volatile(
        "global_load_dword %0, %3, off sc1\n\t"
        "global_load_dword %1, %4, off sc1\n\t"
        "global_load_dword %2, %5, off sc1\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(a), "=&v"(b), "=&v"(c)
        : "v"(p0), "v"(p1), "v"(p2)
        : "memory");
    if (__all((a >> 16) == tag && (b >> 16) == tag && (c >> 16) == tag) || failed || wait_gives_up(n, err))
      break;
  }
  return make_uint3(a & 0xffffu, b & 0xffffu, c & 0xffffu);
}

// ---- k_gdn_xcd: a Gated DeltaNet layer up to its out_proj partials ----
// It replaces the input-norm + projection launch and the recurrence launch.
// XCD x holds the head pair 2x, 2x + 1, 16 blocks each (rank r: head
// 2x + (r >> 4), block j = r & 15 of the head). Phase 1: the layer input
// (embedding row, or the stream after the previous layer's mixer plus its
// MLP's down partials), RMSNorm, and the block's rows of the head: channels
// 8j .. 8j+7 of q, k, v and z (block 0 of the head also a and b), one
// half-wave per row as k_norm_multi; the q/k/v rows go to the ring and
// through the convolution with the ring's three older taps and SiLU.
// Exchange. Phase 2: q and k L2-norms, gates, and the delta rule for value
// rows 8j .. 8j+7 (16 lanes per row, k_gdn_recur_out's order). Exchange.
// Phase 3: both heads' gated RMSNorm and out_proj rows 32r .. 32r+31 over the
// pair's 256 columns: per row tree8 of its eight 32-column slice partials,
// which is the head partial of 2x (tree4 of its four slices) plus that of
// 2x + 1 -- the first level of the pairwise sum over the 16 head partials
// that k_gdn_recur_out writes, so the next launch's pairwise sum of the eight
// pair partials is bit for bit the same.
constexpr int kHx = 648;  // exchange elements per head: q k v z y (128 each), a, b, pad
constexpr int kXq = 0, kXk = 128, kXv = 256, kXz = 384, kXy = 512, kXab = 640;

template <bool EMBED>
__global__ __launch_bounds__(256) void k_gdn_xcd(GdnXcdArgs a) {
  __shared__ float hs[EMBED ? 1 : kNormLds];
  __shared__ float norm_lds[kNormLds];
  __shared__ float qk[256];
  __shared__ float vv[8];
  __shared__ float red[4];
  __shared__ float gates[2];
  __shared__ float yv[256];       // phase 3: y of the head pair
  __shared__ float xg[256 + 8];   // z, then the gated value; slice s at xg[33 s ..]
  __shared__ float ginv[2];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, half = lane >> 5, sl = lane & 31;
  const int hw = wave * 2 + half;  // half-wave 0..7
  const int x = (int)xcc_id() & 7, rank = blockIdx.x >> 3;
  const int h = 2 * x + (rank >> 4), j = rank & 15;
  uint32_t* flags = a.flags + x * kGroupBlocks;
  uint32_t* xb = a.xbuf + (size_t)(x * 2 + (rank >> 4)) * kHx;
  // every pointer argument in scalar registers at once: one wait for the
  // argument fetch instead of one per batch between the vector loads
  asm volatile("" :: "s"(a.x), "s"(a.dpart), "s"(a.h_out), "s"(a.gain), "s"(a.qkv.w), "s"(a.qkv_sb),
               "s"(a.z.w), "s"(a.z_sb), "s"(a.a.w), "s"(a.b.w), "s"(a.ab_sb), "s"(a.out.w), "s"(a.out_sb),
               "s"(a.conv_w), "s"(a.norm_w));
  asm volatile("" :: "s"(a.dt_bias), "s"(a.a_log), "s"(a.ring), "s"(a.state), "s"(a.part), "s"(a.st),
               "s"(a.embed.w), "s"(a.embed.s), "s"(a.embed.b), "s"(a.flags), "s"(a.xbuf), "s"(a.err));

  // ---- loads in the order they are needed: input, gain, position, sense;
  // projection rows; conv taps; state rows; out_proj slice
  const Raw64 graw = EMBED ? load_raw64(a.gain + sl * 32) : Raw64{};
  uint2 x4 = EMBED ? uint2{0u, 0u} : reinterpret_cast<const uint2*>(a.x)[t];
  const uint2 g4 = EMBED ? uint2{0u, 0u} : reinterpret_cast<const uint2*>(a.gain)[t];
  float4 dp[EMBED ? 1 : 8];
  if (!EMBED) {
#pragma unroll
    for (int k = 0; k < 8; ++k) dp[k] = reinterpret_cast<const float4*>(a.dpart + k * kHidden)[t];
  }
  int zero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
  const int pos = (&a.st->pos)[zero];
  const uint32_t own = flags[rank];
  uint32_t err_raw = *a.err;  // set: make no wait (first used at the first exchange)
  // layer 0: the input is the token's embedding row. Its loads go before the
  // weights (loads complete in issue order, so the norm would otherwise wait
  // for every weight load), at the cost of a wait here for the token and the
  // few loads issued before it.
  u32x4 emb_c = {0u, 0u, 0u, 0u};
  uint32_t emb_s = 0u, emb_b = 0u;
  if (EMBED) {
    uint32_t tok = __builtin_amdgcn_readfirstlane((&a.st->token)[zero]);
    if (tok >= (uint32_t)a.embed.n) tok = 0;  // ids come from validated prompts or the head's argmax
    emb_c = *reinterpret_cast<const u32x4*>(a.embed.w + (size_t)tok * 128 + sl * 4);
    emb_s = a.embed.s[(size_t)tok * 16 + sl / 2];
    emb_b = a.embed.b[(size_t)tok * 16 + sl / 2];
  }
  issue_fence();
  // pass p: matrix p (q, k, v rows of in_proj_qkv, then z), channel 8j + hw
  u32x4 c[5];
  uint32_t sbw[5];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int row = (p < 3 ? p * 2048 : 0) + h * 128 + 8 * j + hw;
    c[p] = *reinterpret_cast<const u32x4*>((p < 3 ? a.qkv.w : a.z.w) + (size_t)row * 128 + sl * 4);
    sbw[p] = (p < 3 ? a.qkv_sb : a.z_sb)[(size_t)row * 16 + sl / 2];
  }
  // block 0 of the head: a (half-wave 0) and b (half-wave 1) of the head.
  // The half-waves of a wave differ, so the pointers are chosen per lane from
  // values already in scalar registers (choosing between the two argument
  // structs per lane would read them with vector loads, and waiting for those
  // would also wait for the input loads issued before them).
  const bool ab_pass = j == 0 && hw < 2;
  {
    const bool is_a = hw == 0;
    const int row = ab_pass ? h : 0;
    c[4] = *reinterpret_cast<const u32x4*>((is_a ? a.a.w : a.b.w) + (size_t)row * 128 + sl * 4);
    sbw[4] = a.ab_sb[(size_t)((is_a ? 0 : kGdnHeads) + row) * 16 + sl / 2];
  }
  // conv taps of the half-wave's q, k, v channels (ring slots 0..3) and
  // their conv weights, one load each across the half-wave: lane l < 12
  // holds slot l & 3 of pass l >> 2, lane 12 + p the weights of pass p. The
  // tap is read as the aligned word of channels hw & ~1, hw | 1 (both this
  // block's; element offsets are even up to hw) and its half chosen after the
  // norm: a 16-bit load needs a zero extension the compiler places early.
  const int tl = sl < 12 ? sl : 0, cl = sl >= 12 && sl < 15 ? sl - 12 : 0;
  uint32_t tapw = reinterpret_cast<const uint32_t*>(
      a.ring)[((size_t)(tl & 3) * kConv + (tl >> 2) * 2048 + h * 128 + 8 * j + hw) >> 1];
  const uint2 cwv = *reinterpret_cast<const uint2*>(a.conv_w + (size_t)(cl * 2048 + h * 128 + 8 * j + hw) * 4);
  // per-head constants of phase 2 (lane 8: dt_bias and A_log of the head)
  // and the gated norm's weight of phase 3, loaded now: issued after the
  // exchange loads they would add memory round trips to both phases
  // (unconditional, converted at use: a load under a branch is waited for
  // inside it, and that wait would cover every load issued before it)
  const uint32_t dtb_raw = a.dt_bias[h];
  const float alog = a.a_log[h];
  const uint32_t gnw_raw = a.norm_w[t & 127];
  // state: value rows 8j .. 8j+7 of the head, 16 lanes x 8 keys (t < 128).
  // Read and written non-temporally (1 MB per layer, touched once a step).
  const int srow = 8 * j + (t >> 4) % 8, sj = t & 15;
  float S[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  if (t < 128) {
    const f32x4* sp = reinterpret_cast<const f32x4*>(a.state + ((size_t)(h * 128 + srow)) * 128 + 8 * sj);
    const f32x4 lo = __builtin_nontemporal_load(sp);
    const f32x4 hi = __builtin_nontemporal_load(sp + 1);
    S[0] = lo[0]; S[1] = lo[1]; S[2] = lo[2]; S[3] = lo[3];
    S[4] = hi[0]; S[5] = hi[1]; S[6] = hi[2]; S[7] = hi[3];
  }
  // out_proj: row 32 rank + t/8, K slice 8x + t%8 (the pair's eight slices,
  // 128 contiguous bytes of the row)
  const int orow = 32 * rank + (t >> 3), os8 = t & 7;
  const u32x4 oc = __builtin_nontemporal_load(
      reinterpret_cast<const u32x4*>(a.out.w + (size_t)orow * 256 + (8 * x + os8) * 4));
  const uint32_t osb = __builtin_nontemporal_load(a.out_sb + ((size_t)x * 1024 + orow) * 4 + os8 / 2);
  issue_fence();
  // tags of this launch's two exchanges (q, k, v, z, a, b; then y)
  const uint32_t tag1 = (own + 1u) & 0xffffu, tag2 = (own + 2u) & 0xffffu;

  // ---- phase 1: input, RMSNorm, projection rows, ring, convolution
  float xv[32];
  if (EMBED) {
    embed_convert(emb_c, emb_s, emb_b, xv);
    if (blockIdx.x == 0 && t < 32) store_bf16x32(a.h_out + sl * 32, xv);
  } else {
    const float hf[4] = {bf_lo(x4.x), bf_hi(x4.x), bf_lo(x4.y), bf_hi(x4.y)};
    float hn[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float cc[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) cc[k] = e == 0 ? dp[k].x : e == 1 ? dp[k].y : e == 2 ? dp[k].z : dp[k].w;
      hn[e] = bf2f(f2bf(hf[e] + rbf(((cc[0] + cc[1]) + (cc[2] + cc[3])) + ((cc[4] + cc[5]) + (cc[6] + cc[7])))));
    }
    x4 = make_uint2(pack_bf2(hn[0], hn[1]), pack_bf2(hn[2], hn[3]));
    if (blockIdx.x == 0) reinterpret_cast<uint2*>(a.h_out)[t] = x4;
    *reinterpret_cast<float4*>(hs + (t >> 3) * 36 + (t & 7) * 4) = make_float4(hn[0], hn[1], hn[2], hn[3]);
    __syncthreads();
    const float4* rp = reinterpret_cast<const float4*>(hs + sl * 36);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 q = rp[i];
      xv[4 * i] = q.x; xv[4 * i + 1] = q.y; xv[4 * i + 2] = q.z; xv[4 * i + 3] = q.w;
    }
  }
  float xn[32];
  if (EMBED) norm_slice_1024(xv, graw, xn);
  else norm_block_1024(xv, x4, g4, norm_lds, xn);
  // Keeps work on values loaded late (the conv taps, issued after every
  // projection row) out of the norm: using one there makes the norm wait for
  // all the loads issued before it.
  issue_fence();
  asm volatile("" : "+v"(tapw));
  const uint32_t tapv = (hw & 1) ? tapw >> 16 : tapw & 0xffffu;
  float xr[32];
  const float xs = prep_slice(xn, xr);
  const int slot_new = pos & 3;
  // every lane of a half-wave holds the four projected values (tree32). Lane
  // p < 3 of the half-wave writes pass p's ring row and convolves it over
  // the taps of pos-3 .. pos-1 (ring slots (pos+1+t) & 3, fetched from the
  // lanes that loaded them) and the new row; lane 3 stores z
  const uint32_t raw_q = f2bf(tree32(q4_slice_sb(c[0], sbw[0], xr, xs)));
  const uint32_t raw_k = f2bf(tree32(q4_slice_sb(c[1], sbw[1], xr, xs)));
  const uint32_t raw_v = f2bf(tree32(q4_slice_sb(c[2], sbw[2], xr, xs)));
  const uint32_t raw_z = f2bf(tree32(q4_slice_sb(c[3], sbw[3], xr, xs)));
  {
    const int src = (lane & 32) + 4 * (sl < 3 ? sl : 0);
    const uint32_t x0 = (uint32_t)__shfl((int)tapv, src + ((pos + 1) & 3));
    const uint32_t x1 = (uint32_t)__shfl((int)tapv, src + ((pos + 2) & 3));
    const uint32_t x2 = (uint32_t)__shfl((int)tapv, src + ((pos + 3) & 3));
    const int wsrc = (lane & 32) + 12 + (sl < 3 ? sl : 0);
    const uint2 w = make_uint2((uint32_t)__shfl((int)cwv.x, wsrc), (uint32_t)__shfl((int)cwv.y, wsrc));
    if (sl < 4) {
      const uint32_t raw = sl == 0 ? raw_q : sl == 1 ? raw_k : sl == 2 ? raw_v : raw_z;
      if (sl < 3) {
        a.ring[(size_t)slot_new * kConv + sl * 2048 + h * 128 + 8 * j + hw] = (uint16_t)raw;
        const uint32_t xt[4] = {x0, x1, x2, raw};
        xb[sl * 128 + 8 * j + hw] = f2bf(conv4_silu(xt, w)) | tag1 << 16;  // q, k, v of the exchange
      } else {
        xb[kXz + 8 * j + hw] = raw | tag1 << 16;
      }
    }
  }
  if (j == 0 && wave == 0) {  // wave-uniform: half-waves 0 and 1 form a and b
    const uint32_t raw = f2bf(tree32(q4_slice_sb(c[4], sbw[4], xr, xs)));
    if (sl == 0) xb[kXab + half] = raw | tag1 << 16;
  }
  if (t == 0) flags[rank] = own + 2u;  // this launch's two exchanges

  // ---- phase 2: q/k L2 norms (k_gdn_recur_out's order), gates, delta rule
  // (the error word is used from here on, not at entry: a uniform value
  // formed from a load right after it would wait for every input load before
  // the weights are issued)
  asm volatile("" : "+v"(err_raw));
  const bool failed = err_raw != 0u;
  {
    // lanes 8 and 9 also read a and b (the same exchange), the others their
    // q/k word twice
    const uint32_t* qk_word = xb + (t < 128 ? kXq + t : kXk + (t - 128));
    const uint3 qkr = xcd_poll3(qk_word, xb + kXv + 8 * j + (t & 7), t == 8 || t == 9 ? xb + kXab + (t - 8) : qk_word,
                                tag1, a.err, failed);
    const float v = bf2f(qkr.x);
    const float ss = tree64(v * v);
    if (lane == 0) red[wave] = ss;
    if (t < 8) vv[t] = bf2f(qkr.y);
    if (t == 8) {  // the decay g
      const float ax = rbf(bf2f(qkr.z) + bf2f(dtb_raw));
      gates[0] = es_exp(-es_exp(alog) * softplus_bf(ax));
    } else if (t == 9) {  // beta
      gates[1] = sigmoid_bf(bf2f(qkr.z));
    }
    __syncthreads();
    const float tot = t < 128 ? red[0] + red[1] : red[2] + red[3];
    const float inv = 1.0f / sqrtf(tot / 128.0f + 1.0e-6f / 128.0f);
    const float scale = t < 128 ? 0.0078125f : rbf(0.08838834764831845f);
    qk[t] = rbf(rbf(v * inv) * scale);
    __syncthreads();
  }
  if (t < 128) {  // waves 0 and 1: value rows 8j + t/16
    const float g = gates[0], beta = gates[1];
    float kk[8], qq[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      kk[i] = qk[128 + 8 * sj + i];
      qq[i] = qk[8 * sj + i];
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
    if (sj == 0) xb[kXy + srow] = f2bf(out) | tag2 << 16;
  }

  // ---- phase 3: gated RMSNorm of both heads of the pair (threads 128 hl ..
  // 128 hl + 127: head 2x + hl), out_proj rows 32 rank .. +31
  const int hl = t >> 7, dl = t & 127;
  {
    const uint32_t* xh = a.xbuf + (size_t)(x * 2 + hl) * kHx;
    const uint2 yz = xcd_poll2(xh + kXy + dl, tag2, xh + kXz + dl, tag1, a.err, failed);
    yv[t] = bf2f(yz.x);
    xg[t + (t >> 5)] = bf2f(yz.y);  // z, replaced by the gated value below
  }
  // the updated state rows, stored after the exchange's poll: a store issued
  // before it would hold the poll's wait until the store is acknowledged
  if (t < 128) {
    f32x4* sp = reinterpret_cast<f32x4*>(a.state + ((size_t)(h * 128 + srow)) * 128 + 8 * sj);
    __builtin_nontemporal_store(f32x4{S[0], S[1], S[2], S[3]}, sp);
    __builtin_nontemporal_store(f32x4{S[4], S[5], S[6], S[7]}, sp + 1);
  }
  __syncthreads();
  if (dl < 16) {  // lanes 0-15 of waves 0 and 2
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(yv[128 * hl + dl * 8 + i], yv[128 * hl + dl * 8 + i], ss);
    ss = tree16(ss);
    if (dl == 0) ginv[hl] = 1.0f / sqrtf(ss / 128.0f + 1e-6f);
  }
  __syncthreads();
  {
    const float norm = rbf(rbf(yv[t] * ginv[hl]) * bf2f(gnw_raw));
    const float gz = xg[t + (t >> 5)];
    const float sy = 1.0f / (1.0f + es_exp(fabsf(gz)));
    const float sig = gz < 0.0f ? sy : 1.0f - sy;
    xg[t + (t >> 5)] = rbf((gz * sig) * norm);
  }
  __syncthreads();
  {
    float ov[32], oxr[32];
#pragma unroll
    for (int q = 0; q < 32; ++q) ov[q] = xg[os8 * 33 + q];
    const float oxs = prep_slice(ov, oxr);
    const float part = tree8(q4_slice_sb(oc, osb, oxr, oxs));
    if (os8 == 0) a.part[(size_t)x * 1024 + orow] = part;
  }
}

__global__ __launch_bounds__(256) void k_pack_sb(const uint16_t* s, const uint16_t* b, uint32_t* out, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = (uint32_t)s[i] | (uint32_t)b[i] << 16;
}

__global__ __launch_bounds__(256) void k_pack_sb2(const uint16_t* s0, const uint16_t* b0, const uint16_t* s1,
                                                  const uint16_t* b1, uint2* out, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = make_uint2((uint32_t)s0[i] | (uint32_t)b0[i] << 16, (uint32_t)s1[i] | (uint32_t)b1[i] << 16);
}

// out[x][r][w] for w < 8: groups 4x + w (w < 4), 32 + 4x + w - 4 (w >= 4, x < 6).
__global__ __launch_bounds__(256) void k_pack_down_octets(const uint16_t* s, const uint16_t* b, uint32_t* out) {
  const int i = blockIdx.x * 256 + threadIdx.x;  // < 8 * 1024 * 8
  const int x = i >> 13, r = (i >> 3) & 1023, w = i & 7;
  const int g = w < 4 ? 4 * x + w : 32 + 4 * x + (w - 4);
  const bool used = w < 4 || x < 6;
  const size_t src = (size_t)r * 56 + (used ? g : 0);
  out[i] = used ? ((uint32_t)s[src] | (uint32_t)b[src] << 16) : 0u;
}

// out[x][r][w] = group 4x + w of row r (32 groups per row).
__global__ __launch_bounds__(256) void k_pack_out_pairs(const uint16_t* s, const uint16_t* b, uint32_t* out) {
  const int i = blockIdx.x * 256 + threadIdx.x;  // < 8 * 1024 * 4
  const int x = i >> 12, r = (i >> 2) & 1023, w = i & 3;
  const size_t src = (size_t)r * 32 + 4 * x + w;
  out[i] = (uint32_t)s[src] | (uint32_t)b[src] << 16;
}

__global__ __launch_bounds__(256) void k_xcc_probe(uint32_t* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

}  // namespace

hipError_t launch_mlp_xcd(const MlpXcdArgs& a, int nparts, hipStream_t s) {
  if (!a.gate.w || !a.up.w || !a.down.w || a.gate.k != kHidden || a.up.k != kHidden || a.gate.n != kFfn ||
      a.up.n != kFfn || a.down.n != kHidden || a.down.k != kFfn || !a.h_old || !a.part || !a.h_mid ||
      a.h_mid == a.h_old || !a.gain || !a.dpart || !a.xact || !a.flags || !a.err || !a.gu_sb || !a.down_sb)
    return hipErrorInvalidValue;
  if (nparts != 8) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_mlp_xcd<8>, dim3(256), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_gdn_xcd(const GdnXcdArgs& a, hipStream_t s) {
  const bool embed = a.embed.w != nullptr;
  if (!a.gain || !a.h_out || !a.st || !a.qkv.w || !a.z.w || !a.a.w || !a.b.w || !a.out.w || !a.conv_w ||
      !a.norm_w || !a.dt_bias || !a.a_log || !a.ring || !a.state || !a.part || !a.xbuf || !a.flags || !a.err ||
      !a.qkv_sb || !a.z_sb || !a.ab_sb || !a.out_sb ||
      a.qkv.n != kConv || a.qkv.k != kHidden || a.z.n != 2048 || a.z.k != kHidden || a.a.n != kGdnHeads ||
      a.a.k != kHidden || a.b.n != kGdnHeads || a.b.k != kHidden || a.out.n != kHidden || a.out.k != 2048)
    return hipErrorInvalidValue;
  if (embed ? (a.embed.k != kHidden) : (!a.x || !a.dpart)) return hipErrorInvalidValue;
  if (embed)
    hipLaunchKernelGGL(k_gdn_xcd<true>, dim3(256), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(k_gdn_xcd<false>, dim3(256), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_pack_sb(const uint16_t* s, const uint16_t* b, uint32_t* out, size_t n, hipStream_t st) {
  if (!s || !b || !out || n == 0 || n > ((size_t)1 << 32)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_pack_sb, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, s, b, out, n);
  return hipGetLastError();
}

hipError_t launch_pack_sb2(const uint16_t* s0, const uint16_t* b0, const uint16_t* s1, const uint16_t* b1,
                           uint2* out, size_t n, hipStream_t st) {
  if (!s0 || !b0 || !s1 || !b1 || !out || n == 0 || n > ((size_t)1 << 32)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_pack_sb2, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, s0, b0, s1, b1, out, n);
  return hipGetLastError();
}

hipError_t launch_pack_down_octets(const uint16_t* s, const uint16_t* b, uint32_t* out, hipStream_t st) {
  if (!s || !b || !out) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_pack_down_octets, dim3(8 * 1024 * 8 / 256), dim3(256), 0, st, s, b, out);
  return hipGetLastError();
}

hipError_t launch_pack_out_pairs(const uint16_t* s, const uint16_t* b, uint32_t* out, hipStream_t st) {
  if (!s || !b || !out) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_pack_out_pairs, dim3(8 * 1024 * 4 / 256), dim3(256), 0, st, s, b, out);
  return hipGetLastError();
}

hipError_t launch_xcc_probe(uint32_t* out, hipStream_t s) {
  if (!out) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_xcc_probe, dim3(256), dim3(64), 0, s, out);
  return hipGetLastError();
}

}  // namespace es
