// Decode kernels whose blocks cooperate within one XCD.
//
// MI355X deals the workgroups of a launch to its 8 XCDs in turn, starting
// where the previous launch stopped, so each XCD receives 32 blocks of a
// 256-block launch and the blocks of one XCD have distinct b >> 3. A block
// takes its XCD from the XCC_ID hardware register and its rank within the XCD
// from b >> 3. The 32 blocks of an XCD share its L2 and exchange data through
// it at the cost of one store and one load round trip, where any exchange
// between XCDs costs a kernel boundary. The engine uses these kernels only
// after a start-up probe has seen that dealing. Waits are bounded: a wait that
// exceeds its spin limit (as it would if two blocks of one XCD shared a rank)
// sets an error word, which the engine checks after each batch of steps, and
// the block goes on.
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
constexpr int kSpinLimit = 1 << 22;       // polls before a wait gives up

// Loads that miss the vector L1 and read the XCD's L2, where the stores of the
// group's other blocks land (the L1 writes through).
__device__ __forceinline__ uint32_t l2_load_b32(const void* p) {
  uint32_t v;
  asm volatile("global_load_dword %0, %1, off sc1\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
  return v;
}
// 64 contiguous bytes (four 16-byte loads) the same way. The loads and their
// wait are one statement: the hardware does not hold a read of a register a
// load has not filled yet, so no instruction may touch the outputs before the
// wait.
__device__ __forceinline__ Raw64 l2_load_64B(const void* p) {
  Raw64 r;
  asm volatile(
      "global_load_dwordx4 %0, %4, off sc1\n\t"
      "global_load_dwordx4 %1, %4, off offset:16 sc1\n\t"
      "global_load_dwordx4 %2, %4, off offset:32 sc1\n\t"
      "global_load_dwordx4 %3, %4, off offset:48 sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(r.q[0]), "=&v"(r.q[1]), "=&v"(r.q[2]), "=&v"(r.q[3])
      : "v"(p)
      : "memory");
  return r;
}
__device__ __forceinline__ void wait_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 15u;
}

// Barrier of the 32 blocks of one XCD: every block publishes `sense` in its
// own flag once its stores are in the L2, then waits until all 32 flags carry
// it. Flags alternate between launches, so they never need clearing. Called
// by every thread of the block.
__device__ __forceinline__ void xcd_barrier(uint32_t* flags, int rank, uint32_t sense, uint32_t* err) {
  wait_loads();  // this wave's stores (and loads) are complete
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    if (lane == 0) flags[rank] = sense;
    for (int n = 0;; ++n) {
      const uint32_t f = lane < kGroupBlocks ? l2_load_b32(flags + lane) : sense;
      if (__all(f == sense)) break;
      if (n >= kSpinLimit) {
        if (lane == 0) atomicOr(err, 2u);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
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

  // ---- loads: residual, gain and mixer partials; the sense of this launch;
  // gate/up weights; the down weights of phase 2
  const uint2 ho = reinterpret_cast<const uint2*>(a.h_old)[t];
  const uint2 g4 = reinterpret_cast<const uint2*>(a.gain)[t];
  float4 pv[NPART];
#pragma unroll
  for (int k = 0; k < NPART; ++k) pv[k] = reinterpret_cast<const float4*>(a.part + k * kHidden)[t];
  // this block's flag as it left it in the previous launch (on this XCD)
  const uint32_t own = flags[rank];
  issue_fence();
  u32x4 cg[2], cu[2];
  uint32_t sg[2], bg[2], su[2], bu[2];
  int er[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int j = wave * 4 + 2 * p + half;  // local row in the block
    const int e = j < nact ? octet_act(x, rank * nact + j) : 0;
    er[p] = j < nact ? e : -1;
    cg[p] = *reinterpret_cast<const u32x4*>(a.gate.w + (size_t)e * 128 + sl * 4);
    cu[p] = *reinterpret_cast<const u32x4*>(a.up.w + (size_t)e * 128 + sl * 4);
    sg[p] = a.gate.s[(size_t)e * 16 + sl / 2];
    bg[p] = a.gate.b[(size_t)e * 16 + sl / 2];
    su[p] = a.up.s[(size_t)e * 16 + sl / 2];
    bu[p] = a.up.b[(size_t)e * 16 + sl / 2];
  }
  // phase 2: down rows 32 rank .. +31; x < 6: 16 lanes per row (lane L holds
  // slice 8x+L, or 8x+64+L-8 for L >= 8), two passes of 16 rows; x >= 6: 8
  // lanes per row (slice 8x+L), one pass of 32 rows
  const int wide = x < 6;
  const int L = wide ? (t & 15) : (t & 7);
  const int dslice = wide ? (L < 8 ? 8 * x + L : 8 * x + 64 + (L - 8)) : 8 * x + L;
  u32x4 dc[2];
  uint32_t ds[2], db[2];
  int drow[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int row = wide ? rank * 32 + p * 16 + (t >> 4) : rank * 32 + (t >> 3);
    drow[p] = row;
    dc[p] = *reinterpret_cast<const u32x4*>(a.down.w + (size_t)row * 448 + dslice * 4);
    ds[p] = a.down.s[(size_t)row * 56 + dslice / 2];
    db[p] = a.down.b[(size_t)row * 56 + dslice / 2];
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
  uint16_t* xact = a.xact + x * 512;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const float g = tree32(q4_slice(cg[p], sg[p], bg[p], xr, xs));
    const float u = tree32(q4_slice(cu[p], su[p], bu[p], xr, xs));
    if (sl == 0 && er[p] >= 0) {
      const float gb = rbf(g), ub = rbf(u);
      const float silu = rbf(gb * sigmoid_bf(gb));
      xact[rank * nact + wave * 4 + 2 * p + half] = (uint16_t)f2bf(silu * ub);
    }
  }

  // ---- exchange the XCD's activation elements
  xcd_barrier(flags, rank, own ^ 1u, a.err);

  // ---- phase 2: octet x of every down row of this block
  const int aoff = wide ? (L < 8 ? 32 * L : 256 + 32 * (L - 8)) : 32 * L;
  unpack_bf16x32(l2_load_64B(xact + aoff), xv);
  xs = prep_slice(xv, xr);
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    if (!wide && p == 1) break;
    float v = q4_slice(dc[p], ds[p], db[p], xr, xs);
    if (wide) v = v + dpp_row_ror8(v);  // leaf: slices 8x+L and 8x+64+L
    v = tree4(v);
    v = v + dpp_half_mirror(v);         // the octet's tree over its 8 leaves
    if (L == 0) a.dpart[x * kHidden + drow[p]] = v;
  }
}

__global__ __launch_bounds__(256) void k_xcc_probe(uint32_t* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

}  // namespace

hipError_t launch_mlp_xcd(const MlpXcdArgs& a, int nparts, hipStream_t s) {
  if (!a.gate.w || !a.up.w || !a.down.w || a.gate.k != kHidden || a.up.k != kHidden || a.gate.n != kFfn ||
      a.up.n != kFfn || a.down.n != kHidden || a.down.k != kFfn || !a.h_old || !a.part || !a.h_mid ||
      a.h_mid == a.h_old || !a.gain || !a.dpart || !a.xact || !a.flags || !a.err)
    return hipErrorInvalidValue;
  if (nparts == 16)
    hipLaunchKernelGGL(k_mlp_xcd<16>, dim3(256), dim3(256), 0, s, a);
  else if (nparts == 8)
    hipLaunchKernelGGL(k_mlp_xcd<8>, dim3(256), dim3(256), 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_xcc_probe(uint32_t* out, hipStream_t s) {
  if (!out) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_xcc_probe, dim3(256), dim3(64), 0, s, out);
  return hipGetLastError();
}

}  // namespace es
