// Batched prefill kernels (Model::encode_forward with rows > 1,
// model.rs:228-350): the row-batched forms of the decode path's operators.
//
// k_q4_gemm: Y[M,N] = bf16(X[M,K] . dequant(W)[N,K]^T), optionally
//   Y = bf16(R + that), as qmm_q4_nax (linear_nax.metal:1096-1139) computes
//   it: each weight is dequantised to bf16, bf16(scale*q + bias), and the
//   products accumulate in fp32 (MFMA). Block = 128 rows x 128 features,
//   four waves of 64 x 64, each a 2 x 2 grid of v_mfma_f32_32x32x16_bf16
//   tiles. Per 64-wide K step (one quantisation group) the block stages the
//   X tile and the dequantised W tile in LDS (row stride 72 bf16, so the
//   16-byte fragment reads of 32 rows spread over the banks), double
//   buffered: the next step's global loads are in flight while the current
//   step multiplies.
//   Operand layouts (32x32x16 bf16): lane l holds A[l%32][8(l/32)..+7] and
//   B[8(l/32)..+7][l%32]; result element r of lane l is
//   D[8(r/4) + 4(l/32) + r%4][l%32].
#include "es_kernels.hpp"

namespace es {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Wait until at most N vector-memory operations of this wave are pending.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

constexpr int kGemmBM = 128, kGemmBN = 128, kGemmBK = 64, kGemmLds = 72;

struct GemmStage {
  u32x4 x[4];    // this thread's 64 bytes of the X tile
  u32x4 c;       // 32 nibbles of one W row
  uint32_t s, b; // that row's scale and bias (bf16)
};

// Two values -> packed bf16 pair (lo in bits 0..15), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_bf2(lo, hi); }

// The 8 nibbles of one code word (element j = bits 4j..4j+3) as
// fma(scale, q, bias), packed to four bf16 pairs. The even nibbles are the
// bytes of word & 0x0F0F0F0F and the odd ones the bytes of
// (word >> 4) & 0x0F0F0F0F, so each converts with one v_cvt_f32_ubyteN (the
// masked words are hidden from known-bits analysis, which would otherwise
// extract every nibble separately).
__device__ __forceinline__ u32x4 dequant8(uint32_t word, float sc, float bi) {
  uint32_t lo = word & 0x0F0F0F0Fu;
  uint32_t hi = (word >> 4) & 0x0F0F0F0Fu;
  asm("" : "+v"(lo));
  asm("" : "+v"(hi));
  float v[8];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    v[2 * b] = fmaf(sc, (float)((lo >> (8 * b)) & 0xffu), bi);
    v[2 * b + 1] = fmaf(sc, (float)((hi >> (8 * b)) & 0xffu), bi);
  }
  return u32x4{pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7])};
}

// GATEUP: w is the gate matrix and w2 the up matrix of the MLP; the block's
// 128 staged W rows are gate rows n0 + 0..31, up rows n0 + 0..31, gate rows
// n0 + 32..63, up rows n0 + 32..63, so each wave holds a gate and an up
// accumulator for the same 32 columns and writes
// act = bf16(bf16(g * sigmoid_bf(g)) * u) with g, u the bf16-rounded GEMM
// outputs (swiglu_bf16 after the two linears), y [m, N] with N = w.n.
template <bool GATEUP>
__global__ __launch_bounds__(256) void k_q4_gemm(Q4 w, Q4 w2, const uint16_t* __restrict__ x, int m,
                                                 const uint16_t* residual, uint16_t* y) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][kGemmBM][kGemmLds];
  __shared__ __attribute__((aligned(16))) uint16_t ws[2][kGemmBN][kGemmLds];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n0 = blockIdx.x * (GATEUP ? kGemmBN / 2 : kGemmBN), m0 = blockIdx.y * kGemmBM;
  const int K = w.k, N = w.n;
  const int wpr = K >> 3, gpr = K >> 6;
  // loader roles: X row t/2, 32 columns (t&1); W row t/2, 32 nibbles (t&1)
  const int lr = t >> 1, lh = t & 1;
  const Q4& wsrc = (GATEUP && ((lr >> 5) & 1)) ? w2 : w;
  const int wr = GATEUP ? n0 + (lr >> 6) * 32 + (lr & 31) : n0 + lr;
  const bool xrow_ok = m0 + lr < m, wrow_ok = wr < N;
  const uint16_t* xrow = x + (size_t)(xrow_ok ? m0 + lr : 0) * K + lh * 32;
  const uint32_t* wrow = wsrc.w + (size_t)(wrow_ok ? wr : 0) * wpr + lh * 4;
  const uint16_t* srow = wsrc.s + (size_t)(wrow_ok ? wr : 0) * gpr;
  const uint16_t* brow = wsrc.b + (size_t)(wrow_ok ? wr : 0) * gpr;

  auto load = [&](int kb, GemmStage& g) {
    const u32x4* xp = reinterpret_cast<const u32x4*>(xrow + kb * kGemmBK);
#pragma unroll
    for (int i = 0; i < 4; ++i) g.x[i] = xrow_ok ? xp[i] : u32x4{0u, 0u, 0u, 0u};
    g.c = *reinterpret_cast<const u32x4*>(wrow + kb * 8);
    g.s = srow[kb];
    g.b = brow[kb];
  };
  auto store = [&](int buf, const GemmStage& g) {
    u32x4* xd = reinterpret_cast<u32x4*>(&xs[buf][lr][lh * 32]);
#pragma unroll
    for (int i = 0; i < 4; ++i) xd[i] = g.x[i];
    // dequantise 32 weights to bf16: bf16(fma(scale, q, bias)); rows past N are 0
    const float sc = wrow_ok ? bf2f(g.s) : 0.0f, bi = wrow_ok ? bf2f(g.b) : 0.0f;
    u32x4 o[4];
#pragma unroll
    for (int wd = 0; wd < 4; ++wd) {
      o[wd] = dequant8(g.c[wd], sc, bi);
    }
    u32x4* wd4 = reinterpret_cast<u32x4*>(&ws[buf][lr][lh * 32]);
#pragma unroll
    for (int i = 0; i < 4; ++i) wd4[i] = o[i];
  };

  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int fr = lane & 31, fk = (lane >> 5) * 8;
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nk = K / kGemmBK;
  GemmStage g;
  load(0, g);
  store(0, g);
  __syncthreads();
  for (int kb = 0; kb < nk; ++kb) {
    const int buf = kb & 1;
    if (kb + 1 < nk) load(kb + 1, g);
#pragma unroll
    for (int kk = 0; kk < kGemmBK; kk += 16) {
      bf16x8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const bf16x8*>(&xs[buf][wm + 32 * i + fr][kk + fk]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const bf16x8*>(&ws[buf][wn + 32 * j + fr][kk + fk]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kb + 1 < nk) store(buf ^ 1, g);
    __syncthreads();
  }

  if (GATEUP) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int col = n0 + wn / 2 + fr;
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row >= m) continue;
        const float gb = rbf(acc[i][0][r]), ub = rbf(acc[i][1][r]);
        const float silu = rbf(gb * sigmoid_bf(gb));
        y[(size_t)row * N + col] = (uint16_t)f2bf(silu * ub);
      }
    }
    return;
  }
  // epilogue: bf16 output, or bf16(residual + bf16(acc))
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn + 32 * j + fr;
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row >= m) continue;
        const size_t o = (size_t)row * N + col;
        float v = rbf(acc[i][j][r]);
        if (residual) v = bf2f(residual[o]) + v;
        y[o] = (uint16_t)f2bf(v);
      }
    }
}

// ---- wide GEMM: 256 x 256 block tiles for the linears with N >= 2048 ----
//
// k_q4_gemm_wide computes the same products as k_q4_gemm, bit for bit: the
// same bf16 operands (weights dequantised as bf16(fma(scale, q, bias))) and,
// for every output element, the same sequence of 32x32x16 MFMAs over K in
// increasing order. Only the tiling differs. A block of 256 threads owns a
// 256 x 256 output tile; each wave a 128 x 128 quarter (16 MFMA accumulators
// in the accumulation registers), so every 16-byte fragment read from LDS
// feeds four MFMAs instead of two. X reaches LDS by DMA (global_load_lds, no
// registers); each thread dequantises one weight row per 64-column step.
// LDS rows are 128 bytes with no padding; the 16-byte chunk c of row r sits
// at slot c ^ ((r >> 1) & 7), so the 16 rows that one 16-lane group of a
// fragment read touches cover all 64 banks once. The X DMA applies the same
// permutation on the source side (lane l of an instruction fetches the chunk
// that belongs in its slot).
// Output columns may span up to four weight matrices stacked along N
// (q|k|v, qkv|z|a|b), each written to its own [m][n_s] output.
// A block holds a whole CU (128 KB of LDS, all registers), so beside the
// other prefill stream's recurrence or attention it gets fewer CUs than the
// 128 x 128 kernel, whose blocks share CUs: in the two-stream prefill it pays
// for the stacked input linears (one launch for four) but not for gate/up,
// which keeps k_q4_gemm.
constexpr int kWideM = 256, kWideN = 256, kWideK = 64;

__device__ __forceinline__ int wide_slot(int r, int c) { return ((c ^ ((r >> 1) & 7)) << 3) + (r << 6); }

// Fragment reads as inline assembly: the compiler treats an LDS read after a
// DMA into LDS as dependent on it and would wait for every DMA in flight
// (including the next stage's) before the first read of a step. Four reads
// of one operand: rows r, r+32, r+64, r+96 share the slot, 4096 bytes apart.
__device__ __forceinline__ void wide_read4(uint32_t addr, u32x4& f0, u32x4& f1, u32x4& f2, u32x4& f3) {
  asm volatile(
      "ds_read_b128 %0, %4\n\t"
      "ds_read_b128 %1, %4 offset:4096\n\t"
      "ds_read_b128 %2, %4 offset:8192\n\t"
      "ds_read_b128 %3, %4 offset:12288"
      : "=&v"(f0), "=&v"(f1), "=&v"(f2), "=&v"(f3)
      : "v"(addr));
}
__device__ __forceinline__ void wide_wait8(u32x4 (&a)[4], u32x4 (&b)[4]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]));
}

// One 64-column step of the MFMA loop over the staged tiles at LDS byte
// addresses xt (X) and wt (W): the fragments of slice kk + 1 are read while
// the 16 MFMAs of slice kk run.
__device__ __forceinline__ void wide_step(uint32_t xt, uint32_t wt, int xrow, int wrow, f32x16 (&acc)[4][4],
                                          int fh) {
  // byte address of slot c of rows xrow (+32i) and wrow (+32j)
  auto xaddr = [&](int c) { return xt + (uint32_t)(wide_slot(xrow, c) * 2); };
  auto waddr = [&](int c) { return wt + (uint32_t)(wide_slot(wrow, c) * 2); };
  u32x4 fa[2][4], fb[2][4];
  wide_read4(xaddr(fh), fa[0][0], fa[0][1], fa[0][2], fa[0][3]);
  wide_read4(waddr(fh), fb[0][0], fb[0][1], fb[0][2], fb[0][3]);
  wide_wait8(fa[0], fb[0]);
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int cur = kk & 1;
    if (kk + 1 < 4) {
      const int c = 2 * (kk + 1) + fh;
      wide_read4(xaddr(c), fa[cur ^ 1][0], fa[cur ^ 1][1], fa[cur ^ 1][2], fa[cur ^ 1][3]);
      wide_read4(waddr(c), fb[cur ^ 1][0], fb[cur ^ 1][1], fb[cur ^ 1][2], fb[cur ^ 1][3]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa[cur][i]),
                                                            __builtin_bit_cast(bf16x8, fb[cur][j]), acc[i][j], 0,
                                                            0, 0);
    if (kk + 1 < 4) wide_wait8(fa[cur ^ 1], fb[cur ^ 1]);
  }
}

// Barrier for the staged tiles: the caller has waited for its own X DMA
// (vmcnt); lgkmcnt(0) covers the dequantised weights written by ds_write.
// Unlike __syncthreads it does not wait for the weight loads still in flight.
__device__ __forceinline__ void wide_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The two stages are four separate LDS arrays (not one indexed array), so the
// compiler can see that the DMA into one stage does not write the other and
// does not wait for it before reading fragments.
__shared__ __attribute__((aligned(16))) uint16_t g_wide_x0[kWideM * kWideK];
__shared__ __attribute__((aligned(16))) uint16_t g_wide_x1[kWideM * kWideK];
__shared__ __attribute__((aligned(16))) uint16_t g_wide_w0[kWideN * kWideK];
__shared__ __attribute__((aligned(16))) uint16_t g_wide_w1[kWideN * kWideK];

__global__ __launch_bounds__(256, 1) void k_q4_gemm_wide(WideGemmArgs a) {
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int K = a.w[0].k, m = a.m;
  const int m0 = blockIdx.y * kWideM;
  const int nk = K / kWideK;

  // this thread's weight row: segment, row within it, validity
  const int n_row = blockIdx.x * kWideN + t;
  int seg = 0;
#pragma unroll
  for (int sg = 1; sg < 4; ++sg)
    if (sg < a.nseg && n_row >= a.nstart[sg]) seg = sg;
  const int wrow = n_row - a.nstart[seg];
  const bool wok = n_row < a.nstart[a.nseg];
  const uint32_t* wcodes = seg == 0 ? a.w[0].w : seg == 1 ? a.w[1].w : seg == 2 ? a.w[2].w : a.w[3].w;
  const uint16_t* wsc = seg == 0 ? a.w[0].s : seg == 1 ? a.w[1].s : seg == 2 ? a.w[2].s : a.w[3].s;
  const uint16_t* wbi = seg == 0 ? a.w[0].b : seg == 1 ? a.w[1].b : seg == 2 ? a.w[2].b : a.w[3].b;
  const int r_ok = wok ? wrow : 0;
  const u32x4* cptr = reinterpret_cast<const u32x4*>(wcodes + (size_t)r_ok * (K >> 3));
  const uint16_t* sptr = wsc + (size_t)r_ok * (K >> 6);
  const uint16_t* bptr = wbi + (size_t)r_ok * (K >> 6);

  // X DMA: instruction i of this wave fills LDS rows 8(8w+i) .. +7, lane l
  // the slot l & 7 of row l >> 3
  const int xr_lane = lane >> 3, xslot = lane & 7;
  auto issue_x = [&](int kb, uint16_t* xt) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = (wave * 8 + i) * 8 + xr_lane;
      const int c = xslot ^ ((r >> 1) & 7);
      const int gr = min(m0 + r, m - 1);
      const uint16_t* g = a.x + (size_t)gr * K + kb * kWideK + c * 8;
      __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)&xt[(wave * 8 + i) * 512], 16, 0, 0);
    }
  };
  // Weight loads and the dequantised stores are inline assembly as well, so
  // the compiler inserts no waits of its own in the loop; each wait below is
  // counted by hand (the order of the vector-memory operations of a step:
  // the previous step's 4 weight loads, 8 X DMA, this step's 4 weight loads).
  struct WRegs {
    u32x4 c0, c1;
    uint32_t s, b;
  };
  auto load_w = [&](int kb, WRegs& r) {
    const u32x4* cp = cptr + kb * 2;
    const uint16_t* sp = sptr + kb;
    const uint16_t* bp = bptr + kb;
    asm volatile(
        "global_load_dwordx4 %0, %4, off\n\t"
        "global_load_dwordx4 %1, %4, off offset:16\n\t"
        "global_load_ushort %2, %5, off\n\t"
        "global_load_ushort %3, %6, off"
        : "=&v"(r.c0), "=&v"(r.c1), "=&v"(r.s), "=&v"(r.b)
        : "v"(cp), "v"(sp), "v"(bp));
  };
  // dequantise 64 weights (bf16(fma(scale, q, bias)); rows past N are 0);
  // the caller has waited for the set's loads
  auto store_w = [&](uint32_t wt, const WRegs& r) {
    const float sc = wok ? bf2f(r.s) : 0.0f, bi = wok ? bf2f(r.b) : 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const u32x4 o = dequant8(c < 4 ? r.c0[c] : r.c1[c - 4], sc, bi);
      asm volatile("ds_write_b128 %0, %1" ::"v"(wt + (uint32_t)(wide_slot(t, c) * 2)), "v"(o));
    }
  };
  // waits for a weight set with N vector-memory operations issued after it
  auto wait_set12 = [](WRegs& r) { asm volatile("s_waitcnt vmcnt(12)" : "+v"(r.c0), "+v"(r.c1), "+v"(r.s), "+v"(r.b)); };
  auto wait_set4 = [](WRegs& r) { asm volatile("s_waitcnt vmcnt(4)" : "+v"(r.c0), "+v"(r.c1), "+v"(r.s), "+v"(r.b)); };

  const int wm = (wave >> 1) * 128, wn = (wave & 1) * 128;
  const int fr = lane & 31, fh = lane >> 5;
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // Weights are loaded two steps ahead (register sets wa, wb) and dequantised
  // into the stage being filled while the MFMAs of the other stage run; the
  // end-of-step wait covers the X DMA but not the four weight loads issued
  // after it.
  auto lds_addr = [](const uint16_t* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)p;
  };
  const uint32_t lx0 = lds_addr(g_wide_x0), lx1 = lds_addr(g_wide_x1);
  const uint32_t lw0 = lds_addr(g_wide_w0), lw1 = lds_addr(g_wide_w1);
  // Weights are loaded two steps ahead (register set wa for even steps, wb
  // for odd) and dequantised into the stage being filled after the MFMAs of
  // the other stage are issued. Every step issues the same operations, so the
  // loop has no branch between a load and its wait: the X DMA of step s + 1
  // (8 operations) and the weight loads of step s + 2 (4), with the step
  // clamped to the last one (those loads fill the stage nobody reads again).
  // At the start of step s only the loads of weight set s + 1 are in flight;
  // it waits for them with 12 operations issued after them, and for its DMA
  // with 4.
  WRegs wa, wb;
  issue_x(0, g_wide_x0);
  load_w(0, wa);
  load_w(1, wb);
  wait_set4(wa);
  store_w(lw0, wa);
  wide_barrier();
  auto run_step = [&](int st, uint32_t lx, uint32_t lw, uint16_t* x_next, uint32_t lw_next, WRegs& w_next,
                      WRegs& w_after) {
    issue_x(min(st + 1, nk - 1), x_next);
    load_w(min(st + 2, nk - 1), w_after);
    issue_fence();
    wide_step(lx, lw, wm + fr, wn + fr, acc, fh);
    wait_set12(w_next);
    store_w(lw_next, w_next);
    wait_vmcnt<4>();
    wide_barrier();
  };
  for (int kb = 0; kb < nk; kb += 2) {  // K is a multiple of 128: nk even
    run_step(kb, lx0, lw0, g_wide_x1, lw1, wb, wa);
    run_step(kb + 1, lx1, lw1, g_wide_x0, lw0, wa, wb);
  }
  // The last step's weight loads (into wb) are still in flight: wait with
  // both sets as operands, so the compiler keeps their registers until the
  // data has landed instead of giving them to the epilogue.
  asm volatile("s_waitcnt vmcnt(0)"
               : "+v"(wa.c0), "+v"(wa.c1), "+v"(wa.s), "+v"(wa.b), "+v"(wb.c0), "+v"(wb.c1), "+v"(wb.s), "+v"(wb.b));

#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = blockIdx.x * kWideN + wn + 32 * j + fr;
    if (n >= a.nstart[a.nseg]) continue;
    int sg = 0;
#pragma unroll
    for (int q = 1; q < 4; ++q)
      if (q < a.nseg && n >= a.nstart[q]) sg = q;
    uint16_t* y = sg == 0 ? a.y[0] : sg == 1 ? a.y[1] : sg == 2 ? a.y[2] : a.y[3];
    const int ld = a.nstart[sg + 1] - a.nstart[sg], col = n - a.nstart[sg];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * fh + (r & 3);
        if (row < m) y[(size_t)row * ld + col] = (uint16_t)f2bf(acc[i][j][r]);
      }
  }
}

// ---- row kernels: the decode operators' arithmetic, one row per token ----

// Embedding rows (embedding_q4, linear.metal:11-24): h = bf16(scale*q + bias).
// Half-wave per row, 32 elements per lane.
__global__ __launch_bounds__(256) void k_embed_rows(Q4 e, const uint32_t* tokens, int m, uint16_t* h) {
  const int row = blockIdx.x * 8 + (threadIdx.x >> 5), sl = threadIdx.x & 31;
  if (row >= m) return;
  uint32_t tok = tokens[row];
  if (tok >= (uint32_t)e.n) tok = 0;
  const u32x4 c = *reinterpret_cast<const u32x4*>(e.w + (size_t)tok * 128 + sl * 4);
  const float sc = bf2f(e.s[(size_t)tok * 16 + sl / 2]), bi = bf2f(e.b[(size_t)tok * 16 + sl / 2]);
  float xv[32];
#pragma unroll
  for (int w = 0; w < 4; ++w)
#pragma unroll
    for (int j = 0; j < 8; ++j) xv[8 * w + j] = rbf(fmaf(sc, (float)((c[w] >> (4 * j)) & 15u), bi));
  store_bf16x32(h + (size_t)row * 1024 + sl * 32, xv);
}

// RMSNorm rows (rms_norm_bf16 rounding points, the decode kernels' order).
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const uint16_t* x, const uint16_t* gain, int m,
                                                      uint16_t* out) {
  const int row = blockIdx.x * 8 + (threadIdx.x >> 5), sl = threadIdx.x & 31;
  if (row >= m) return;
  const Raw64 xr = load_raw64(x + (size_t)row * 1024 + sl * 32);
  const Raw64 gr = load_raw64(gain + sl * 32);
  float xv[32], xn[32];
  unpack_bf16x32(xr, xv);
  norm_slice_1024(xv, gr, xn);
  store_bf16x32(out + (size_t)row * 1024 + sl * 32, xn);
}

// SwiGLU (swiglu_bf16, linear.metal:382-398): silu = bf16(g*sigmoid_bf(g)),
// act = bf16(silu*up), over bf16 gate and up.
__global__ __launch_bounds__(256) void k_swiglu_rows(const uint16_t* gate, const uint16_t* up, int count,
                                                     uint16_t* act) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  const float gb = bf2f(gate[i]), ub = bf2f(up[i]);
  const float silu = rbf(gb * sigmoid_bf(gb));
  act[i] = (uint16_t)f2bf(silu * ub);
}

// GDN prepare rows (gdn_conv + gdn_prepare, gdn.metal:33-120, with the decode
// kernels' arithmetic): one wave per (4 consecutive rows, head), which loads
// the 7 input rows the 4 rows' taps span once. Lane i takes channels i and
// 64+i of the head's q, k and v: causal conv over taps (pos-3 .. pos) whose
// inputs are the chunk's raw rows, or the ring for positions before the
// chunk; SiLU; q and k L2-normalised (sum of squares tree64 over channels
// 0..63 plus tree64 over 64..127) and scaled (q by 1/128, k by bf16(128^-1/2));
// lane 0 forms the gates g = exp(-exp(A_log)*softplus(bf16(a+dt))), beta =
// sigmoid_bf(b). Outputs bf16 q, k, v [m,16,128] and fp32 g, beta [m,16].
constexpr int kPrepRows = 4;  // rows per wave: their taps span kPrepRows + 3 input rows
__global__ __launch_bounds__(256) void k_gdn_prep_rows(const uint16_t* raw, const uint16_t* ring,
                                                       const uint16_t* conv_w, const uint16_t* a_proj,
                                                       const uint16_t* b_proj, const float* a_log,
                                                       const uint16_t* dt_bias, int pos0, int m,
                                                       uint16_t* q, uint16_t* k, uint16_t* v, float* g,
                                                       float* beta) {
  const int lane = threadIdx.x & 63, h = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int t0 = blockIdx.x * kPrepRows;
  if (t0 >= m) return;
  const int nr = min(kPrepRows, m - t0);
  float out[3][2][kPrepRows];
#pragma unroll
  for (int part = 0; part < 3; ++part)
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int c = part * 2048 + h * 128 + half * 64 + lane;
      // input rows t0-3 .. t0+kPrepRows-1: the chunk's raw rows, or the ring
      // for positions before the chunk; rows past the chunk are not used
      uint32_t x[kPrepRows + 3];
#pragma unroll
      for (int i = 0; i < kPrepRows + 3; ++i) {
        const int tt = t0 - 3 + i;
        x[i] = tt >= 0 ? (tt < m ? raw[(size_t)tt * kConv + c] : 0u)
                       : ring[(size_t)((pos0 + tt) & 3) * kConv + c];
      }
      const uint2 w = *reinterpret_cast<const uint2*>(conv_w + (size_t)c * 4);
#pragma unroll
      for (int r = 0; r < kPrepRows; ++r) out[part][half][r] = conv4_silu(x + r, w);
    }
#pragma unroll
  for (int r = 0; r < kPrepRows; ++r) {
    if (r >= nr) break;
    const int t = t0 + r;
    const size_t o = ((size_t)t * 16 + h) * 128;
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      const float tot = tree64(out[part][0][r] * out[part][0][r]) + tree64(out[part][1][r] * out[part][1][r]);
      const float inv = 1.0f / sqrtf(tot / 128.0f + 1.0e-6f / 128.0f);
      const float scale = part == 0 ? 0.0078125f : rbf(0.08838834764831845f);
      uint16_t* dst = part == 0 ? q : k;
      dst[o + lane] = (uint16_t)f2bf(rbf(out[part][0][r] * inv) * scale);
      dst[o + 64 + lane] = (uint16_t)f2bf(rbf(out[part][1][r] * inv) * scale);
    }
    v[o + lane] = (uint16_t)f2bf(out[2][0][r]);
    v[o + 64 + lane] = (uint16_t)f2bf(out[2][1][r]);
    if (lane == 0) {
      const float ax = rbf(bf2f(a_proj[(size_t)t * 16 + h]) + bf2f(dt_bias[h]));
      g[(size_t)t * 16 + h] = es_exp(-es_exp(a_log[h]) * softplus_bf(ax));
      beta[(size_t)t * 16 + h] = sigmoid_bf(bf2f(b_proj[(size_t)t * 16 + h]));
    }
  }
}

// History after a chunk (gdn_history, gdn.metal:56-73, as the decode ring):
// the raw rows of the chunk's last min(m, 4) positions go to slot pos & 3.
__global__ __launch_bounds__(256) void k_ring_update(const uint16_t* raw, int pos0, int m, uint16_t* ring) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int r = i / kConv, c = i % kConv;
  const int t = m - 4 + r;
  if (r >= 4 || t < 0) return;
  ring[(size_t)((pos0 + t) & 3) * kConv + c] = raw[(size_t)t * kConv + c];
}

// The reference's GDN interface kernels over a history [3, 6144] (oldest row
// first, GDN_INTERFACE.md:12-18), with the arithmetic of the kernels above.
// gdn_conv (gdn.metal:31-51): conv [T,6144] = SiLU(bf16(4-tap conv)), taps
// before the first row from the history.
__global__ __launch_bounds__(256) void k_gdn_conv_hist(const uint16_t* raw, const uint16_t* history,
                                                       const uint16_t* conv_w, int rows, uint16_t* conv) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * kConv) return;
  const int t = i / kConv, c = i % kConv;
  uint32_t x[4];
#pragma unroll
  for (int tap = 0; tap < 4; ++tap) {
    const int r = t + tap - 3;
    x[tap] = r < 0 ? history[(size_t)(r + 3) * kConv + c] : raw[(size_t)r * kConv + c];
  }
  conv[i] = (uint16_t)f2bf(conv4_silu(x, *reinterpret_cast<const uint2*>(conv_w + (size_t)c * 4)));
}

// gdn_history (gdn.metal:53-73): the history takes the last three raw rows,
// keeping older history rows when rows < 3.
__global__ __launch_bounds__(256) void k_gdn_history(const uint16_t* raw, int rows, uint16_t* history) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= kConv) return;
  const uint16_t h0 = history[c], h1 = history[kConv + c], h2 = history[2 * kConv + c];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int r = rows + j - 3;  // row j of the new history; r < 0 keeps history row r + 3
    const uint16_t keep = r == -3 ? h0 : r == -2 ? h1 : h2;
    history[(size_t)j * kConv + c] = r < 0 ? keep : raw[(size_t)r * kConv + c];
  }
}

// gdn_prepare (gdn.metal:75-114): one wave per (row, head) normalises the
// head's q and k in place in conv (lane i: channels i and 64 + i, sum of
// squares tree64 + tree64, as k_gdn_prep_rows) and lane 0 forms g (fp32) and
// beta (bf16).
__global__ __launch_bounds__(256) void k_gdn_prepare_hist(uint16_t* conv, const uint16_t* a_proj,
                                                          const uint16_t* b_proj, const float* a_log,
                                                          const uint16_t* dt_bias, int rows, float* g,
                                                          uint16_t* beta) {
  const int lane = threadIdx.x & 63;
  const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= rows * 16) return;
  const int t = wid >> 4, h = wid & 15;
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    uint16_t* p = conv + (size_t)t * kConv + part * 2048 + h * 128;
    const float x0 = bf2f(p[lane]), x1 = bf2f(p[64 + lane]);
    const float tot = tree64(x0 * x0) + tree64(x1 * x1);
    const float inv = 1.0f / sqrtf(tot / 128.0f + 1.0e-6f / 128.0f);
    const float scale = part == 0 ? 0.0078125f : rbf(0.08838834764831845f);
    p[lane] = (uint16_t)f2bf(rbf(x0 * inv) * scale);
    p[64 + lane] = (uint16_t)f2bf(rbf(x1 * inv) * scale);
  }
  if (lane == 0) {
    const float ax = rbf(bf2f(a_proj[wid]) + bf2f(dt_bias[h]));
    g[wid] = es_exp(-es_exp(a_log[h]) * softplus_bf(ax));
    beta[wid] = (uint16_t)f2bf(sigmoid_bf(bf2f(b_proj[wid])));
  }
}

// GDN recurrence over the rows of a chunk (gdn_recur with rows > 1,
// gdn.metal:176-228), the decode kernel's arithmetic and order per token:
// block = (16 value rows, head), thread = (row, 8 keys), state in registers
// for the whole chunk. Tokens go through LDS in tiles of 64, double
// buffered: the next tile's global loads are issued before the current tile
// is walked and land in the other buffer after it, one barrier per tile.
// Within a tile the next token's operands are read from LDS while the
// current token's chain runs. Lane j of a row keeps the readout of tokens
// with index j mod 16 and stores them 16 tokens at a time.
constexpr int kRecurTile = 64;
struct RecurTileRegs {
  u32x4 q[4], k[4];
  uint2 v;
  float gb;
};
// q, k, v rows are `ld` elements apart (2048 for [m,16,128] arrays, 6144 for
// the reference's normalised conv buffer [T,6144]); beta is fp32 or, when
// beta_bf is set, the reference's bf16 [T,16].
struct RecurIn {
  const uint16_t *q, *k, *v;
  int ld;
  const float* g;
  const float* beta;
  const uint16_t* beta_bf;
};
__device__ __forceinline__ void recur_tile_load(const RecurIn& in, int h, int r0, int t0, int nt,
                                                RecurTileRegs& R) {
  const int t = threadIdx.x;
  const int tt = t >> 2, c = (t & 3) * 32;
  if (tt < nt) {
    const size_t o = (size_t)(t0 + tt) * in.ld + h * 128 + c;
    const u32x4* qp = reinterpret_cast<const u32x4*>(in.q + o);
    const u32x4* kp = reinterpret_cast<const u32x4*>(in.k + o);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      R.q[i] = qp[i];
      R.k[i] = kp[i];
    }
    R.v = *reinterpret_cast<const uint2*>(in.v + (size_t)(t0 + tt) * in.ld + h * 128 + r0 + (t & 3) * 4);
  }
  if (t < 2 * kRecurTile && (t & 63) < nt) {
    const size_t gi = (size_t)(t0 + (t & 63)) * 16 + h;
    R.gb = t < 64 ? in.g[gi] : in.beta_bf ? bf2f(in.beta_bf[gi]) : in.beta[gi];
  }
}
// LDS tile rows: 132 floats apart (the 16 rows a store instruction covers
// fall in different banks); within a row, channel c of 8-channel group j sits
// at 4j + (c & 3), plus 64 for the group's upper four, so the two 16-byte
// reads of a row's 16 lanes each cover 256 contiguous bytes.
constexpr int kRecurRow = 132;
__device__ __forceinline__ void recur_tile_store(const RecurTileRegs& R, int nt, float (*qs)[kRecurRow],
                                                 float (*ks)[kRecurRow], float (*vs)[16], float (*gs)[2]) {
  const int t = threadIdx.x;
  const int tt = t >> 2, j0 = (t & 3) * 4;
  if (tt < nt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int jj = j0 + i;
      *reinterpret_cast<float4*>(&qs[tt][4 * jj]) =
          make_float4(bf_lo(R.q[i][0]), bf_hi(R.q[i][0]), bf_lo(R.q[i][1]), bf_hi(R.q[i][1]));
      *reinterpret_cast<float4*>(&qs[tt][64 + 4 * jj]) =
          make_float4(bf_lo(R.q[i][2]), bf_hi(R.q[i][2]), bf_lo(R.q[i][3]), bf_hi(R.q[i][3]));
      *reinterpret_cast<float4*>(&ks[tt][4 * jj]) =
          make_float4(bf_lo(R.k[i][0]), bf_hi(R.k[i][0]), bf_lo(R.k[i][1]), bf_hi(R.k[i][1]));
      *reinterpret_cast<float4*>(&ks[tt][64 + 4 * jj]) =
          make_float4(bf_lo(R.k[i][2]), bf_hi(R.k[i][2]), bf_lo(R.k[i][3]), bf_hi(R.k[i][3]));
    }
    const int rr = (t & 3) * 4;
    vs[tt][rr] = bf_lo(R.v.x);
    vs[tt][rr + 1] = bf_hi(R.v.x);
    vs[tt][rr + 2] = bf_lo(R.v.y);
    vs[tt][rr + 3] = bf_hi(R.v.y);
  }
  if (t < 2 * kRecurTile && (t & 63) < nt) gs[t & 63][t >> 6] = R.gb;
}
__global__ __launch_bounds__(256, 1) void k_gdn_recur_rows(RecurIn in, int m, float* state, uint16_t* y) {
  __shared__ __attribute__((aligned(16))) float qs[2][kRecurTile][kRecurRow];
  __shared__ __attribute__((aligned(16))) float ks[2][kRecurTile][kRecurRow];
  __shared__ float vs[2][kRecurTile][16];
  __shared__ float gs[2][kRecurTile][2];
  // blockIdx.x = head, blockIdx.y = block of 16 value rows: the dispatcher
  // deals consecutive blocks to the 8 XCDs in turn, so the 8 row blocks of a
  // head land on one XCD and share its L2 copy of the head's q and k
  const int t = threadIdx.x, h = blockIdx.x, r0 = blockIdx.y * 16;
  const int rl = t >> 4, row = r0 + rl, j = t & 15;
  float* sp = state + ((size_t)(h * 128 + row)) * 128 + 8 * j;
  const float4 s_lo = reinterpret_cast<const float4*>(sp)[0];
  const float4 s_hi = reinterpret_cast<const float4*>(sp)[1];
  float S[8] = {s_lo.x, s_lo.y, s_lo.z, s_lo.w, s_hi.x, s_hi.y, s_hi.z, s_hi.w};
  RecurTileRegs R;
  recur_tile_load(in, h, r0, 0, min(kRecurTile, m), R);
  recur_tile_store(R, min(kRecurTile, m), qs[0], ks[0], vs[0], gs[0]);
  __syncthreads();
  uint16_t* yrow = y + h * 128 + row;
  for (int t0 = 0, buf = 0; t0 < m; t0 += kRecurTile, buf ^= 1) {
    const int nt = min(kRecurTile, m - t0);
    const int nt_next = min(kRecurTile, m - t0 - kRecurTile);
    if (nt_next > 0) recur_tile_load(in, h, r0, t0 + kRecurTile, nt_next, R);
    // one token: lane j of the row keeps the readout of token index j
    // within its group of 16; its operands are read one token ahead
    struct TokOps {
      float4 k0, k1, q0, q1;
      float2 gb;
      float v;
    };
    auto operands = [&](int tt) {
      TokOps o;
      o.k0 = *reinterpret_cast<const float4*>(&ks[buf][tt][4 * j]);
      o.k1 = *reinterpret_cast<const float4*>(&ks[buf][tt][64 + 4 * j]);
      o.q0 = *reinterpret_cast<const float4*>(&qs[buf][tt][4 * j]);
      o.q1 = *reinterpret_cast<const float4*>(&qs[buf][tt][64 + 4 * j]);
      o.gb = *reinterpret_cast<const float2*>(&gs[buf][tt][0]);
      o.v = vs[buf][tt][rl];
      return o;
    };
    auto token = [&](const TokOps& o, int u, float& keep) {
      const float kk[8] = {o.k0.x, o.k0.y, o.k0.z, o.k0.w, o.k1.x, o.k1.y, o.k1.z, o.k1.w};
      const float qq[8] = {o.q0.x, o.q0.y, o.q0.z, o.q0.w, o.q1.x, o.q1.y, o.q1.z, o.q1.w};
      float mem = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        S[i] = S[i] * o.gb.x;
        mem = fmaf(S[i], kk[i], mem);
      }
      mem = tree16(mem);
      const float delta = (o.v - mem) * o.gb.y;
      float out = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        S[i] = fmaf(kk[i], delta, S[i]);
        out = fmaf(S[i], qq[i], out);
      }
      out = tree16(out);
      keep = u == j ? out : keep;
    };
    for (int g0 = 0; g0 < nt; g0 += 16) {
      const int n16 = min(16, nt - g0);
      float keep = 0.0f;
      if (n16 == 16) {
        TokOps cur = operands(g0);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          TokOps nxt;
          if (u + 1 < 16) nxt = operands(g0 + u + 1);
          token(cur, u, keep);
          cur = nxt;
        }
      } else {
        for (int u = 0; u < n16; ++u) token(operands(g0 + u), u, keep);
      }
      if (j < n16) yrow[(size_t)(t0 + g0 + j) * 2048] = (uint16_t)f2bf(keep);
    }
    if (nt_next > 0) recur_tile_store(R, nt_next, qs[buf ^ 1], ks[buf ^ 1], vs[buf ^ 1], gs[buf ^ 1]);
    __syncthreads();
  }
  reinterpret_cast<float4*>(sp)[0] = make_float4(S[0], S[1], S[2], S[3]);
  reinterpret_cast<float4*>(sp)[1] = make_float4(S[4], S[5], S[6], S[7]);
}

// GDN gated norm rows (gdn_norm_gate, gdn.metal:230-255, the decode kernels'
// arithmetic): 16 lanes per (row, head), 8 channels per lane: sum of squares
// as an fma chain per lane then tree16; out = bf16(SiLU_fp32(z) *
// bf16(bf16(y*inv)*w)). One block per row (16 heads).
__global__ __launch_bounds__(256) void k_gdn_norm_gate_rows(const uint16_t* y, const uint16_t* z,
                                                            const uint16_t* norm_w, int m, uint16_t* out) {
  const int t = blockIdx.x, h = threadIdx.x >> 4, li = threadIdx.x & 15;
  if (t >= m) return;
  const size_t o = (size_t)t * 2048 + h * 128 + li * 8;
  const uint4 yr = *reinterpret_cast<const uint4*>(y + o);
  const uint4 zr = *reinterpret_cast<const uint4*>(z + o);
  const uint4 wr = *reinterpret_cast<const uint4*>(norm_w + li * 8);
  const uint32_t yw[4] = {yr.x, yr.y, yr.z, yr.w}, zw[4] = {zr.x, zr.y, zr.z, zr.w}, ww[4] = {wr.x, wr.y, wr.z, wr.w};
  float yv[8], zv[8], wv[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    yv[2 * i] = bf_lo(yw[i]); yv[2 * i + 1] = bf_hi(yw[i]);
    zv[2 * i] = bf_lo(zw[i]); zv[2 * i + 1] = bf_hi(zw[i]);
    wv[2 * i] = bf_lo(ww[i]); wv[2 * i + 1] = bf_hi(ww[i]);
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = fmaf(yv[i], yv[i], ss);
  ss = tree16(ss);
  const float ginv = 1.0f / sqrtf(ss / 128.0f + 1e-6f);
  uint32_t res[4];
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    float r2[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float norm = rbf(rbf(yv[i + u] * ginv) * wv[i + u]);
      const float gz = zv[i + u];
      const float sy = 1.0f / (1.0f + es_exp(fabsf(gz)));
      const float sig = gz < 0.0f ? sy : 1.0f - sy;
      r2[u] = rbf((gz * sig) * norm);
    }
    res[i / 2] = pack_bf2(r2[0], r2[1]);
  }
  *reinterpret_cast<uint4*>(out + o) = make_uint4(res[0], res[1], res[2], res[3]);
}

// Attention prepare rows (attn_prepare_q / attn_prepare_kv,
// attention.metal:72-131, with the decode kernel's arithmetic): one wave per
// (row, q head) for q, per (row, kv head) for k (RMSNorm, RoPE at position
// pos0 + row) and v; k and v rows go to the cache. Block = one row, 12 waves.
__global__ __launch_bounds__(768) void k_attn_prep_rows(const uint16_t* qg, const uint16_t* kp,
                                                        const uint16_t* vp, const uint16_t* q_gain,
                                                        const uint16_t* k_gain, const float* inv_freq,
                                                        int pos0, int m, uint16_t* qr, uint16_t* kcache,
                                                        uint16_t* vcache, int capacity) {
  const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (t >= m) return;
  const int pos = pos0 + t;
  if (wave >= 10) {  // v rows of the two kv heads
    const int kvh = wave - 10;
    const uint2 xv = *reinterpret_cast<const uint2*>(vp + (size_t)t * 512 + kvh * 256 + lane * 4);
    *reinterpret_cast<uint2*>(vcache + ((size_t)kvh * capacity + pos) * 256 + lane * 4) = xv;
    return;
  }
  uint2 xv, gv;
  if (wave < 8) {
    xv = *reinterpret_cast<const uint2*>(qg + (size_t)t * 4096 + wave * 512 + lane * 4);
    gv = *reinterpret_cast<const uint2*>(q_gain + lane * 4);
  } else {
    xv = *reinterpret_cast<const uint2*>(kp + (size_t)t * 512 + (wave - 8) * 256 + lane * 4);
    gv = *reinterpret_cast<const uint2*>(k_gain + lane * 4);
  }
  float inv[4];
#pragma unroll
  for (int x = 0; x < 4; ++x) inv[x] = inv_freq[((lane * 4) & 31) + x];
  float o4[4], p4[4], r[4];
  head_norm4(xv, gv, o4);
#pragma unroll
  for (int x = 0; x < 4; ++x) p4[x] = dpp_row_ror8(o4[x]);
#pragma unroll
  for (int x = 0; x < 4; ++x) r[x] = rope_at(o4[x], p4[x], lane * 4 + x, pos, inv[x]);
  const uint2 packed = make_uint2(pack_bf2(r[0], r[1]), pack_bf2(r[2], r[3]));
  if (wave < 8)
    *reinterpret_cast<uint2*>(qr + ((size_t)t * 8 + wave) * 256 + lane * 4) = packed;
  else
    *reinterpret_cast<uint2*>(kcache + ((size_t)(wave - 8) * capacity + pos) * 256 + lane * 4) = packed;
}

// Output gate rows (attn_gate, attention.metal:133-151): gated =
// bf16(o * sigmoid_bf(gate)) with o the bf16 attention output and gate the
// second half of each head's q_proj row.
__global__ __launch_bounds__(256) void k_attn_gate_rows(const uint16_t* o, const uint16_t* qg, int m,
                                                        uint16_t* gated) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= m * 2048) return;
  const int t = i >> 11, hd = i & 2047, h = hd >> 8, d = hd & 255;
  const float gate = sigmoid_bf(bf2f(qg[(size_t)t * 4096 + h * 512 + 256 + d]));
  gated[i] = (uint16_t)f2bf(bf2f(o[i]) * gate);
}

// Causal GQA attention of m consecutive queries (positions pos0 .. pos0+m-1)
// over the cache (attn_prefill, attention_prefill.metal:2256; model.rs:337-343):
// o = bf16(softmax(q.K^T / 16) . V), fp32 softmax, MFMA products.
// Block = (32 queries, KV head), 8 waves, two per SIMD: wave w serves query
// head 4*kvh + (w & 3) for queries 16(w >> 2) .. +15 of the tile. Per block of
// 32 keys, S^T = K . Q^T on 16x16x32 MFMAs (two 16-key tiles, K from LDS, the
// wave's Q fragments in registers): lane l holds 8 scores of query l%16, keys
// 4g + r and 16 + 4g + r (g = l/16, r = 0..3), so the online-softmax max and
// sum combine 4 lanes with two row exchanges. The exp'ed scores, rounded to
// bf16, are directly the B operand of O^T += V^T . P^T, with the MFMA's k index
// 8g + j standing for key (j < 4 ? 4g + j : 16 + 4g + j - 4). Exponentials are
// base 2 on scores scaled by log2(e)/16.
//
// K and V blocks reach LDS by DMA (global_load_lds, 16 bytes a lane, no
// registers), kFaStages blocks deep: block kb + kFaStages - 1 is issued while
// block kb is computed. One DMA instruction moves one 512-byte row (32
// lanes); K rows sit 528 bytes apart and V rows 544 bytes apart, strides at
// which the K reads (16 rows x 4 chunks) and the transposing V reads
// (ds_read_b64_tr_b16: 16 rows x 32 bytes) spread evenly over the banks. The
// transposing read gives lane i of each 16-lane group element i of the 4 rows
// x 16 columns its lanes address: lane l gets V[4 keys][d = 16t + l%16]. It is
// issued as inline assembly with its own lgkmcnt wait, which keeps the
// compiler from waiting for every DMA in flight before it.
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kFaQ = 32, kFaStages = 4, kFaKs = 264, kFaVs = 272;
constexpr int kFaStageHalves = 32 * kFaKs + 32 * kFaVs;
// sixteen transposing reads from one base: eight at OFF + 32*i (keys 4g..)
// and eight at kFaHi + OFF + 32*i (keys 16 + 4g..). At most 15 LDS operations
// are in flight (the width of lgkmcnt): the last read of the second set is
// issued once the first eight have landed. Every read completes before the
// statement ends.
constexpr int kFaHi = 2 * 16 * kFaVs;  // bytes from key row 4g to key row 16 + 4g
template <int OFF>
__device__ __forceinline__ void lds_read_tr16_x16(uint32_t a, uint2 (&ra)[8], uint2 (&rb)[8]) {
  uint64_t x0, x1, x2, x3, x4, x5, x6, x7, y0, y1, y2, y3, y4, y5, y6, y7;
  asm volatile(
      "ds_read_b64_tr_b16 %0, %16 offset:%17\n\t"
      "ds_read_b64_tr_b16 %1, %16 offset:%17+32\n\t"
      "ds_read_b64_tr_b16 %2, %16 offset:%17+64\n\t"
      "ds_read_b64_tr_b16 %3, %16 offset:%17+96\n\t"
      "ds_read_b64_tr_b16 %4, %16 offset:%17+128\n\t"
      "ds_read_b64_tr_b16 %5, %16 offset:%17+160\n\t"
      "ds_read_b64_tr_b16 %6, %16 offset:%17+192\n\t"
      "ds_read_b64_tr_b16 %7, %16 offset:%17+224\n\t"
      "ds_read_b64_tr_b16 %8, %16 offset:%18\n\t"
      "ds_read_b64_tr_b16 %9, %16 offset:%18+32\n\t"
      "ds_read_b64_tr_b16 %10, %16 offset:%18+64\n\t"
      "ds_read_b64_tr_b16 %11, %16 offset:%18+96\n\t"
      "ds_read_b64_tr_b16 %12, %16 offset:%18+128\n\t"
      "ds_read_b64_tr_b16 %13, %16 offset:%18+160\n\t"
      "ds_read_b64_tr_b16 %14, %16 offset:%18+192\n\t"
      "s_waitcnt lgkmcnt(7)\n\t"
      "ds_read_b64_tr_b16 %15, %16 offset:%18+224\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3), "=&v"(x4), "=&v"(x5), "=&v"(x6), "=&v"(x7),
        "=&v"(y0), "=&v"(y1), "=&v"(y2), "=&v"(y3), "=&v"(y4), "=&v"(y5), "=&v"(y6), "=&v"(y7)
      : "v"(a), "n"(OFF), "n"(kFaHi + OFF)
      : "memory");
  ra[0] = __builtin_bit_cast(uint2, x0);
  ra[1] = __builtin_bit_cast(uint2, x1);
  ra[2] = __builtin_bit_cast(uint2, x2);
  ra[3] = __builtin_bit_cast(uint2, x3);
  ra[4] = __builtin_bit_cast(uint2, x4);
  ra[5] = __builtin_bit_cast(uint2, x5);
  ra[6] = __builtin_bit_cast(uint2, x6);
  ra[7] = __builtin_bit_cast(uint2, x7);
  rb[0] = __builtin_bit_cast(uint2, y0);
  rb[1] = __builtin_bit_cast(uint2, y1);
  rb[2] = __builtin_bit_cast(uint2, y2);
  rb[3] = __builtin_bit_cast(uint2, y3);
  rb[4] = __builtin_bit_cast(uint2, y4);
  rb[5] = __builtin_bit_cast(uint2, y5);
  rb[6] = __builtin_bit_cast(uint2, y6);
  rb[7] = __builtin_bit_cast(uint2, y7);
}
// max of two scores by v_max_f32 alone: scores are never NaN, so the operand
// canonicalisation that fmaxf adds changes nothing and is left out
__device__ __forceinline__ float max_raw(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__global__ __launch_bounds__(512, 1) void k_attn_prefill(const uint16_t* qr, const uint16_t* kcache,
                                                         const uint16_t* vcache, int pos0, int m,
                                                         int capacity, uint16_t* o) {
  __shared__ __attribute__((aligned(16))) uint16_t kv[kFaStages][kFaStageHalves];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: scalar DMA addressing
  // 1-D grid dealt to the 8 XCDs in turn (block b on XCD b % 8): XCDs
  // 0, 2, 4, 6 take KV head 0 and 1, 3, 5, 7 head 1, so the query tiles that
  // stream one head's K and V share an XCD's L2
  const int b = blockIdx.x, xcd = b & 7;
  const int tile = 4 * (b >> 3) + (xcd >> 1);
  if (tile * kFaQ >= m) return;
  const int t0 = tile * kFaQ, kvh = xcd & 1, hq = 4 * kvh + (wave & 3);
  const int qi = lane & 15, g = lane >> 4;
  const int qrow = t0 + 16 * (wave >> 2) + qi;
  const bool qvalid = qrow < m;
  const int qpos = pos0 + (qvalid ? qrow : m - 1);
  const int last_key = pos0 + min(t0 + kFaQ, m) - 1;
  const int nkb = last_key / 32 + 1;
  // Q fragments: B operand of k-step s holds Q[q][32s + 8g .. +7]
  bf16x8 qf[8];
  {
    const uint16_t* qp = qr + ((size_t)(qvalid ? qrow : 0) * 8 + hq) * 256 + 8 * g;
#pragma unroll
    for (int s2 = 0; s2 < 8; ++s2) {
      u32x4 v = *reinterpret_cast<const u32x4*>(qp + 32 * s2);
      if (!qvalid) v = u32x4{0u, 0u, 0u, 0u};
      qf[s2] = __builtin_bit_cast(bf16x8, v);
    }
  }
  // DMA of one block of 32 keys: wave w moves rows 4w .. 4w+3 of K and V,
  // one row per instruction, lane L < 32 the row's 16-byte chunk L
  // Buffer resources over this KV head's rows of both caches: the row's byte
  // offset is a scalar operand and the lane's 16-byte chunk a fixed vector
  // offset, so a DMA takes no per-lane address arithmetic. Rows are clamped
  // to the capacity below, which the launcher keeps at most 2^22 (byte
  // offsets up to 2^31), so the resources set no range of their own.
  const size_t head_off = (size_t)kvh * capacity * 256;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)(kcache + head_off), 0, -1, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)(vcache + head_off), 0, -1, 0x00020000);
  const uint32_t lane_off = (uint32_t)lane * 16u;
  auto issue = [&](int kb) {
    uint16_t* stage = kv[kb % kFaStages];
    if (lane < 32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * wave + i;
        const int key = min(kb * 32 + r, capacity - 1);
        const uint32_t row = (uint32_t)key * 512u;  // uniform byte offset
        __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (__attribute__((address_space(3))) void*)(stage + r * kFaKs), 16,
                                             lane_off, row, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (__attribute__((address_space(3))) void*)(stage + 32 * kFaKs + r * kFaVs),
                                             16, lane_off, row, 0, 0);
      }
    }
  };
  for (int kb = 0; kb < min(kFaStages - 1, nkb); ++kb) issue(kb);
  f32x4 ot[16];
#pragma unroll
  for (int dt = 0; dt < 16; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) ot[dt][r] = 0.0f;
  float mrun = -INFINITY, lrun = 0.0f;
  const float c = 0.0625f * 1.4426950408889634f;  // 1/16 * log2(e)
  // V read roles (see above): lane address row K0 + (l%16)/4, columns
  // 4((l%16)%4) of the first 16-dim tile, K0 = 4g (keys of k indices 0..3)
  // or 16 + 4g (k indices 4..7)
  const uint32_t kv_base =
      (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) uint16_t*)(&kv[0][0]));
  const uint32_t v_lane = (uint32_t)(2 * (32 * kFaKs + (4 * g + (qi >> 2)) * kFaVs + 4 * (qi & 3)));
  for (int kb = 0; kb < nkb; ++kb) {
    // blocks issued after kb and still in flight: min(kFaStages - 2, nkb-1-kb),
    // 8 DMA instructions each per wave
    const int ahead = min(kFaStages - 2, nkb - 1 - kb);
    if (ahead >= 2)
      wait_vmcnt<16>();
    else if (ahead == 1)
      wait_vmcnt<8>();
    else
      wait_vmcnt<0>();
    __syncthreads();  // block kb visible; every wave is past block kb-1
    const uint16_t* ks = kv[kb % kFaStages];
    const uint32_t vs_addr = kv_base + (uint32_t)(2 * kFaStageHalves * (kb % kFaStages)) + v_lane;
    // scores S^T[key][q] for the two 16-key tiles of this block
    // The K fragments of k-steps s2 .. s2 + 3 are in flight while step s2's
    // two products run (fences keep the order), so each pair of products
    // waits for its own reads only.
    f32x4 st[2];
    {
      bf16x8 kf[2][8];
      auto read_k = [&](int s2) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
          kf[kt][s2] = *reinterpret_cast<const bf16x8*>(ks + (16 * kt + qi) * kFaKs + 32 * s2 + 8 * g);
      };
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) read_k(s2);
      // block kb + 3 goes to the stage every wave finished before the barrier;
      // its DMA is issued while the first K reads are in flight
      if (kb + kFaStages - 1 < nkb) issue(kb + kFaStages - 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) st[kt][r] = 0.0f;
#pragma unroll
      for (int s2 = 0; s2 < 8; ++s2) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
          st[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kt][s2], qf[s2], st[kt], 0, 0, 0);
        if (s2 + 4 < 8) read_k(s2 + 4);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    float x[8];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) x[4 * kt + r] = st[kt][r];
    // causal mask (only blocks that reach past the tile's first query),
    // online softmax for query qi; the maximum is taken on the raw scores
    // (scaling by c > 0 keeps the order) and the exponent is fma(s, c, -max)
    if (kb * 32 + 31 > pos0 + t0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = kb * 32 + 16 * (e >> 2) + 4 * g + (e & 3);
        x[e] = key <= qpos ? x[e] : -INFINITY;
      }
    }
    float mloc = x[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mloc = fmaxf(mloc, x[e]);
    const float2 m16 = rows_xor16(mloc);
    const float2 m32 = rows_xor32(max_raw(m16.x, m16.y));
    // The exponent's reference value moves only when the block's maximum
    // exceeds it by more than 8 (probabilities stay below 2^8; the output is
    // normalised by a sum taken against the same reference, so the softmax is
    // unchanged). The choice is per row, so a row's result depends on its own
    // scores only.
    const float mblk = max_raw(m32.x, m32.y) * c;
    const float mnew = mblk > mrun + 8.0f ? mblk : mrun;
    const float factor = __builtin_amdgcn_exp2f(mrun - mnew);
    float pv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[e] = __builtin_amdgcn_exp2f(fmaf(x[e], c, -mnew));
    // ((p0 + p1) + p2) + ...: the same sum as from 0, since p0 >= +0
    float psum = pv[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) psum += pv[e];
    const float2 s16 = rows_xor16(psum);
    const float2 s32 = rows_xor32(s16.x + s16.y);
    lrun = lrun * factor + (s32.x + s32.y);
    const float mrun_old = mrun;
    mrun = mnew;
    // factor is exactly 1 where the reference did not move: the rescale is
    // skipped unless some lane's reference moved
    if (__any(mnew > mrun_old)) {
#pragma unroll
      for (int dt = 0; dt < 16; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) ot[dt][r] *= factor;
    }
    // O^T += V^T . P^T: one 32-key step per 16-dim tile
    const u32x4 pb = u32x4{pack2(pv[0], pv[1]), pack2(pv[2], pv[3]), pack2(pv[4], pv[5]), pack2(pv[6], pv[7])};
    const bf16x8 pf = __builtin_bit_cast(bf16x8, pb);
#pragma unroll
    for (int d8 = 0; d8 < 2; ++d8) {
      uint2 lo[8], hi[8];
      if (d8 == 0)
        lds_read_tr16_x16<0>(vs_addr, lo, hi);
      else
        lds_read_tr16_x16<256>(vs_addr, lo, hi);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int dt = 8 * d8 + i;
        const bf16x8 vf = __builtin_bit_cast(bf16x8, u32x4{lo[i].x, lo[i].y, hi[i].x, hi[i].y});
        ot[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, ot[dt], 0, 0, 0);
      }
    }
  }
  if (!qvalid) return;
  const float inv = 1.0f / lrun;
  uint16_t* op = o + ((size_t)qrow * 8 + hq) * 256 + 4 * g;
#pragma unroll
  for (int dt = 0; dt < 16; ++dt)
    *reinterpret_cast<uint2*>(op + 16 * dt) =
        make_uint2(pack2(ot[dt][0] * inv, ot[dt][1] * inv), pack2(ot[dt][2] * inv, ot[dt][3] * inv));
}

}  // namespace

// The wide kernel takes a GEMM whose total N fills at least eight of its
// 256-column tiles; narrower ones (N = 1024 and below, with the residual add)
// keep the 128 x 128 tiles, which give 256 or more blocks.
static bool wide_ok(int n_total, int k) { return n_total >= 8 * kWideN && k % (2 * kWideK) == 0; }

static hipError_t launch_wide(const WideGemmArgs& a, hipStream_t s) {
  const dim3 grid((a.nstart[a.nseg] + kWideN - 1) / kWideN, (a.m + kWideM - 1) / kWideM);
  hipLaunchKernelGGL(k_q4_gemm_wide, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_q4_gemm_stacked(const Q4* w, uint16_t* const* y, int nseg, const uint16_t* x, int m,
                                  hipStream_t s) {
  if (!w || !y || nseg < 1 || nseg > 4 || !x || m < 1) return hipErrorInvalidValue;
  WideGemmArgs a{};
  int n = 0;
  for (int i = 0; i < nseg; ++i) {
    if (!w[i].w || !w[i].s || !w[i].b || !y[i] || w[i].n < 1 || w[i].k != w[0].k || w[i].k < kGemmBK ||
        w[i].k % kGemmBK != 0)
      return hipErrorInvalidValue;
    a.w[i] = w[i];
    a.y[i] = y[i];
    a.nstart[i] = n;
    n += w[i].n;
  }
  for (int i = nseg; i < 4; ++i) {
    a.w[i] = w[0];
    a.y[i] = y[0];
  }
  a.nstart[nseg] = n;
  for (int i = nseg + 1; i < 5; ++i) a.nstart[i] = n;
  a.nseg = nseg;
  a.x = x;
  a.m = m;
  if (wide_ok(n, w[0].k)) return launch_wide(a, s);
  for (int i = 0; i < nseg; ++i) {
    const dim3 grid((w[i].n + kGemmBN - 1) / kGemmBN, (m + kGemmBM - 1) / kGemmBM);
    hipLaunchKernelGGL(k_q4_gemm<false>, grid, dim3(256), 0, s, w[i], w[i], x, m, nullptr, y[i]);
  }
  return hipGetLastError();
}

hipError_t launch_q4_gemm(const Q4& w, const uint16_t* x, int m, const uint16_t* residual, uint16_t* y,
                          hipStream_t s) {
  if (!w.w || !w.s || !w.b || w.n < 1 || w.k < kGemmBK || w.k % kGemmBK != 0 || !x || !y || m < 1)
    return hipErrorInvalidValue;
  if (!residual && wide_ok(w.n, w.k)) return launch_q4_gemm_stacked(&w, &y, 1, x, m, s);
  const dim3 grid((w.n + kGemmBN - 1) / kGemmBN, (m + kGemmBM - 1) / kGemmBM);
  hipLaunchKernelGGL(k_q4_gemm<false>, grid, dim3(256), 0, s, w, w, x, m, residual, y);
  return hipGetLastError();
}

hipError_t launch_q4_gemm_swiglu(const Q4& gate, const Q4& up, const uint16_t* x, int m, uint16_t* act,
                                 hipStream_t s) {
  if (!gate.w || !gate.s || !gate.b || !up.w || !up.s || !up.b || gate.n != up.n || gate.k != up.k ||
      gate.n < 1 || gate.k < kGemmBK || gate.k % kGemmBK != 0 || !x || !act || m < 1)
    return hipErrorInvalidValue;
  const dim3 grid((gate.n + kGemmBN / 2 - 1) / (kGemmBN / 2), (m + kGemmBM - 1) / kGemmBM);
  hipLaunchKernelGGL(k_q4_gemm<true>, grid, dim3(256), 0, s, gate, up, x, m, nullptr, act);
  return hipGetLastError();
}

}  // namespace es

namespace es {

hipError_t launch_embed_rows(const Q4& e, const uint32_t* tokens, int m, uint16_t* h, hipStream_t s) {
  if (!e.w || m < 1 || !tokens || !h || e.k != 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_embed_rows, dim3((m + 7) / 8), dim3(256), 0, s, e, tokens, m, h);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_rows(const uint16_t* x, const uint16_t* gain, int m, uint16_t* out, hipStream_t s) {
  if (!x || !gain || !out || m < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_rmsnorm_rows, dim3((m + 7) / 8), dim3(256), 0, s, x, gain, m, out);
  return hipGetLastError();
}

hipError_t launch_swiglu_rows(const uint16_t* gate, const uint16_t* up, int count, uint16_t* act,
                              hipStream_t s) {
  if (!gate || !up || !act || count < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_swiglu_rows, dim3((count + 255) / 256), dim3(256), 0, s, gate, up, count, act);
  return hipGetLastError();
}

hipError_t launch_gdn_prep_rows(const GdnPrepRowsArgs& a, hipStream_t s) {
  if (!a.raw || !a.ring || !a.conv_w || !a.a_proj || !a.b_proj || !a.a_log || !a.dt_bias || a.m < 1 ||
      a.pos0 < 0 || !a.q || !a.k || !a.v || !a.g || !a.beta)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gdn_prep_rows, dim3((a.m + kPrepRows - 1) / kPrepRows, 4), dim3(256), 0, s, a.raw, a.ring,
                     a.conv_w, a.a_proj, a.b_proj, a.a_log, a.dt_bias, a.pos0, a.m, a.q, a.k, a.v, a.g, a.beta);
  if (hipGetLastError() != hipSuccess) return hipErrorLaunchFailure;
  hipLaunchKernelGGL(k_ring_update, dim3((4 * kConv + 255) / 256), dim3(256), 0, s, a.raw, a.pos0, a.m,
                     a.ring);
  return hipGetLastError();
}

hipError_t launch_gdn_recur_rows(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                                 const float* beta, int m, float* state, uint16_t* y, hipStream_t s) {
  if (!q || !k || !v || !g || !beta || !state || !y || m < 1) return hipErrorInvalidValue;
  const RecurIn in{q, k, v, 2048, g, beta, nullptr};
  hipLaunchKernelGGL(k_gdn_recur_rows, dim3(kGdnHeads, 8), dim3(256), 0, s, in, m, state, y);
  return hipGetLastError();
}

hipError_t launch_gdn_conv_hist(const uint16_t* raw, const uint16_t* history, const uint16_t* conv_w,
                                int rows, uint16_t* conv, hipStream_t s) {
  if (!raw || !history || !conv_w || !conv || rows < 1 || rows > (1 << 18)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gdn_conv_hist, dim3((rows * kConv + 255) / 256), dim3(256), 0, s, raw, history, conv_w,
                     rows, conv);
  return hipGetLastError();
}

hipError_t launch_gdn_history(const uint16_t* raw, int rows, uint16_t* history, hipStream_t s) {
  if (!raw || !history || rows < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gdn_history, dim3(kConv / 256), dim3(256), 0, s, raw, rows, history);
  return hipGetLastError();
}

hipError_t launch_gdn_prepare_hist(uint16_t* conv, const uint16_t* a_proj, const uint16_t* b_proj,
                                   const float* a_log, const uint16_t* dt_bias, int rows, float* g,
                                   uint16_t* beta, hipStream_t s) {
  if (!conv || !a_proj || !b_proj || !a_log || !dt_bias || !g || !beta || rows < 1 || rows > (1 << 24))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gdn_prepare_hist, dim3((rows * 16 + 3) / 4), dim3(256), 0, s, conv, a_proj, b_proj, a_log,
                     dt_bias, rows, g, beta);
  return hipGetLastError();
}

hipError_t launch_gdn_recur_conv(const uint16_t* conv, const float* g, const uint16_t* beta, int rows,
                                 float* state, uint16_t* y, hipStream_t s) {
  if (!conv || !g || !beta || !state || !y || rows < 1) return hipErrorInvalidValue;
  const RecurIn in{conv, conv + 2048, conv + 4096, kConv, g, nullptr, beta};
  hipLaunchKernelGGL(k_gdn_recur_rows, dim3(kGdnHeads, 8), dim3(256), 0, s, in, rows, state, y);
  return hipGetLastError();
}

hipError_t launch_gdn_norm_gate_rows(const uint16_t* y, const uint16_t* z, const uint16_t* norm_w, int m,
                                     uint16_t* out, hipStream_t s) {
  if (!y || !z || !norm_w || !out || m < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gdn_norm_gate_rows, dim3(m), dim3(256), 0, s, y, z, norm_w, m, out);
  return hipGetLastError();
}

hipError_t launch_attn_prep_rows(const AttnPrepRowsArgs& a, hipStream_t s) {
  if (!a.qg || !a.k || !a.v || !a.q_gain || !a.k_gain || !a.inv_freq || a.m < 1 || a.pos0 < 0 ||
      a.pos0 + a.m > a.capacity || !a.qr || !a.kcache || !a.vcache)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_prep_rows, dim3(a.m), dim3(768), 0, s, a.qg, a.k, a.v, a.q_gain, a.k_gain,
                     a.inv_freq, a.pos0, a.m, a.qr, a.kcache, a.vcache, a.capacity);
  return hipGetLastError();
}

hipError_t launch_attn_prefill(const uint16_t* qr, const uint16_t* kcache, const uint16_t* vcache, int pos0,
                               int m, int capacity, uint16_t* o, hipStream_t s) {
  // capacity <= 2^22 (the engine's limit) keeps every byte offset within a KV
  // head's rows below 2^31
  if (!qr || !kcache || !vcache || !o || m < 1 || pos0 < 0 || pos0 + m > capacity || capacity > (1 << 22))
    return hipErrorInvalidValue;
  const int tiles = (m + kFaQ - 1) / kFaQ;
  hipLaunchKernelGGL(k_attn_prefill, dim3(8 * ((tiles + 3) / 4)), dim3(512), 0, s, qr, kcache, vcache, pos0, m,
                     capacity, o);
  return hipGetLastError();
}

hipError_t launch_attn_gate_rows(const uint16_t* o, const uint16_t* qg, int m, uint16_t* gated,
                                 hipStream_t s) {
  if (!o || !qg || !gated || m < 1 || m > (1 << 20) - 1) return hipErrorInvalidValue;  // m * 2048 < 2^31
  hipLaunchKernelGGL(k_attn_gate_rows, dim3((m * 2048 + 255) / 256), dim3(256), 0, s, o, qg, m, gated);
  return hipGetLastError();
}

}  // namespace es
