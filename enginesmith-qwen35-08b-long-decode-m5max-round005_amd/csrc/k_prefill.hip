// Batched prefill kernels (Model::encode_forward with rows > 1,
// model.rs:228-350): the row-batched forms of the decode path's operators.
//
// k_q4_gemm: Y[M,N] = bf16(X[M,K] . dequant(W)[N,K]^T), optionally
//   Y = bf16(R + that), as qmm_q4_nax (linear_nax.metal:1096-1140) computes
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

constexpr int kGemmBM = 128, kGemmBN = 128, kGemmBK = 64, kGemmLds = 72;

struct GemmStage {
  u32x4 x[4];    // this thread's 64 bytes of the X tile
  u32x4 c;       // 32 nibbles of one W row
  uint32_t s, b; // that row's scale and bias (bf16)
};

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}

__global__ __launch_bounds__(256) void k_q4_gemm(Q4 w, const uint16_t* __restrict__ x, int m,
                                                 const uint16_t* residual, uint16_t* y) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][kGemmBM][kGemmLds];
  __shared__ __attribute__((aligned(16))) uint16_t ws[2][kGemmBN][kGemmLds];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n0 = blockIdx.x * kGemmBN, m0 = blockIdx.y * kGemmBM;
  const int K = w.k, N = w.n;
  const int wpr = K >> 3, gpr = K >> 6;
  // loader roles: X row t/2, 32 columns (t&1); W row t/2, 32 nibbles (t&1)
  const int lr = t >> 1, lh = t & 1;
  const bool xrow_ok = m0 + lr < m, wrow_ok = n0 + lr < N;
  const uint16_t* xrow = x + (size_t)(xrow_ok ? m0 + lr : 0) * K + lh * 32;
  const uint32_t* wrow = w.w + (size_t)(wrow_ok ? n0 + lr : 0) * wpr + lh * 4;
  const uint16_t* srow = w.s + (size_t)(wrow_ok ? n0 + lr : 0) * gpr;
  const uint16_t* brow = w.b + (size_t)(wrow_ok ? n0 + lr : 0) * gpr;

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
      const uint32_t c = g.c[wd];
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = fmaf(sc, (float)((c >> (4 * j)) & 15u), bi);
      o[wd] = u32x4{pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7])};
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

}  // namespace

hipError_t launch_q4_gemm(const Q4& w, const uint16_t* x, int m, const uint16_t* residual, uint16_t* y,
                          hipStream_t s) {
  if (!w.w || !w.s || !w.b || w.n < 1 || w.k < kGemmBK || w.k % kGemmBK != 0 || !x || !y || m < 1)
    return hipErrorInvalidValue;
  const dim3 grid((w.n + kGemmBN - 1) / kGemmBN, (m + kGemmBM - 1) / kGemmBM);
  hipLaunchKernelGGL(k_q4_gemm, grid, dim3(256), 0, s, w, x, m, residual, y);
  return hipGetLastError();
}

}  // namespace es
