// Final RMSNorm + tied Q4 vocab head + log-sum-exp + greedy pick.
//
// k_head: each block of 256 threads computes 256 consecutive logits (a wave
// owns 64 rows, two per pass, loads double-buffered four passes at a time),
// rounds them to bf16 (head_lse.metal:53) and writes its own (max, sum exp)
// over those bf16 logits: max exact, sum = (t0 + t1) + (t2 + t3) of the four
// waves' tree64 sums of exp(logit - max).
// k_head_tail (one block) merges the partials into
//   lse = bf16(log(sum) + max)                         (head_lse.metal:81)
// where thread t sums blocks t, t+256, ... sequentially (each term
// sum_b * exp(max_b - max)), then the four waves' tree64 sums are added as
// (t0 + t1) + (t2 + t3),
// and selects the lowest index whose bf16(logit - lse) equals the maximum
// (head_lse.metal:83-97, docs/protocol.md:44). Rounding is monotone, so the
// maximum is bf16(maxlogit - lse), and the lowest block whose own maximum
// reaches it holds the answer. The tail also advances the device cursor.
#include "es_kernels.hpp"

#include <mutex>

namespace es {
namespace {

constexpr int kRowsPerBlock = 256;
constexpr int kPassBatch = 4;  // passes (2 rows each) whose loads are in flight together
constexpr int kBatches = 64 / (2 * kPassBatch);

__device__ __forceinline__ unsigned int wave_umin(unsigned int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned int o = (unsigned int)__shfl_xor((int)v, off, 64);
    v = o < v ? o : v;
  }
  return v;
}

struct HeadBatch {
  u32x4 c[kPassBatch];
  uint32_t s[kPassBatch], b[kPassBatch];
};

// Buffer resources over the codes, scales and biases of the table: rows past
// the vocabulary are out of range and read as zero, so no row is clamped, and
// the per-row offsets are immediates on one per-lane base offset. The table
// (143 MB, read once per step) is read non-temporally so it does not evict
// the layer weights from the on-package cache.
struct HeadRsrc {
  __amdgpu_buffer_rsrc_t w, s, b;
};

__device__ __forceinline__ void head_load(const HeadRsrc& rs, int voff_c, int voff_s, int it,
                                          HeadBatch& hb) {
#pragma unroll
  for (int p = 0; p < kPassBatch; ++p) {
    const int dr = it * 2 * kPassBatch + 2 * p;  // rows past the lane's first row
    hb.c[p] = __builtin_amdgcn_raw_buffer_load_b128(rs.w, voff_c + dr * 512, 0, kLoadNonTemporal);
    hb.s[p] = __builtin_amdgcn_raw_buffer_load_b16(rs.s, voff_s + dr * 32, 0, kLoadNonTemporal);
    hb.b[p] = __builtin_amdgcn_raw_buffer_load_b16(rs.b, voff_s + dr * 32, 0, kLoadNonTemporal);
  }
}

// Block (max, sum exp) over the 256 bf16 logits held one per thread (-inf
// past the vocabulary): max exact, sum = (t0 + t1) + (t2 + t3) of the four
// waves' tree64 sums of exp(logit - max).
__device__ __forceinline__ void block_lse_part(float v, float* wred, float* wred2, float* part) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  float bm = wave_max(v);
  if (lane == 0) wred[wave] = bm;
  __syncthreads();
  bm = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
  const float se = tree64(v == -INFINITY ? 0.0f : es_exp(v - bm));
  if (lane == 0) wred2[wave] = se;
  __syncthreads();
  if (t == 0) {
    part[2 * blockIdx.x] = bm;
    part[2 * blockIdx.x + 1] = (wred2[0] + wred2[1]) + (wred2[2] + wred2[3]);
  }
}

template <bool PARTS>
__global__ __launch_bounds__(256) void k_head(HeadArgs a) {
  __shared__ float lg[kRowsPerBlock];
  __shared__ float wred[4];
  __shared__ float wred2[4];
  __shared__ float norm_lds[kNormLds];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, half = lane >> 5, sl = lane & 31;
  const int vocab = a.embed.n;
  const int row0 = blockIdx.x * kRowsPerBlock + wave * 64;
  const HeadRsrc rs{
      __builtin_amdgcn_make_buffer_rsrc((void*)a.embed.w, 0, vocab * 512, 0x00020000),
      __builtin_amdgcn_make_buffer_rsrc((void*)a.embed.s, 0, vocab * 32, 0x00020000),
      __builtin_amdgcn_make_buffer_rsrc((void*)a.embed.b, 0, vocab * 32, 0x00020000)};
  const int voff_c = (row0 + half) * 512 + sl * 16;
  const int voff_s = (row0 + half) * 32 + (sl >> 1) * 2;

  HeadBatch cur, nxt;
  head_load(rs, voff_c, voff_s, 0, cur);

  // normalised input slice (rms_norm_bf16 with the final norm gain)
  const Raw64 xraw = PARTS ? Raw64{} : load_raw64(a.h + sl * 32);
  uint2 x4 = reinterpret_cast<const uint2*>(a.h)[t];
  const uint2 g4 = reinterpret_cast<const uint2*>(a.gain)[t];
  float4 dp[PARTS ? 8 : 1];
  if (PARTS) {
#pragma unroll
    for (int k = 0; k < 8; ++k) dp[k] = reinterpret_cast<const float4*>(a.dpart + k * kHidden)[t];
  }
  issue_fence();
  float xv[32], xn[32], xr[32];
  if (PARTS) {
    // h = bf16(h + bf16(pairwise sum of the down projection's octet partials))
    __shared__ float hs[kNormLds];
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
  norm_block_1024(xv, x4, g4, norm_lds, xn);
  if (a.norm_out && blockIdx.x == 0 && t < 32) {
#pragma unroll
    for (int i = 0; i < 32; ++i) a.norm_out[sl * 32 + i] = (uint16_t)f2bf(xn[i]);
  }
  const float xs = prep_slice(xn, xr);

#pragma unroll
  for (int it = 0; it < kBatches; ++it) {
    if (it + 1 < kBatches) head_load(rs, voff_c, voff_s, it + 1, nxt);
#pragma unroll
    for (int p = 0; p < kPassBatch; ++p) {
      const int local = wave * 64 + it * 2 * kPassBatch + 2 * p + half;
      const int r = blockIdx.x * kRowsPerBlock + local;
      const float part = tree32(q4_slice(cur.c[p], cur.s[p], cur.b[p], xr, xs));
      if (sl == 0) {
        const uint32_t b = f2bf(part);
        lg[local] = r < vocab ? bf2f(b) : -INFINITY;
        if (r < vocab) a.logits[r] = (uint16_t)b;
      }
    }
    if (it + 1 < kBatches) cur = nxt;
  }
  __syncthreads();
  block_lse_part(lg[t], wred, wred2, a.part);
}

// greedy_bf16's first stage (linear.metal:400-449) over logits in memory:
// the (max, sum exp) of each block of 256, in k_head's order. The second
// stage is k_head_tail.
__global__ __launch_bounds__(256) void k_logits_part(const uint16_t* logits, int count, float* part) {
  __shared__ float wred[4];
  __shared__ float wred2[4];
  const int r = blockIdx.x * kRowsPerBlock + threadIdx.x;
  block_lse_part(r < count ? bf2f(logits[r]) : -INFINITY, wred, wred2, part);
}

__global__ __launch_bounds__(256) void k_head_tail(HeadArgs a, int nb) {
  __shared__ float wred[4];
  __shared__ float wred2[4];
  __shared__ unsigned int wmin[4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int vocab = a.embed.n;
  // Thread t's block partials (blocks t, t + 256, ...) are read once into
  // registers when there are at most kTailRegs of them (the model's
  // vocabulary needs 4), instead of once per pass; the step state too.
  constexpr int kTailRegs = 4;
  const bool in_regs = nb <= 256 * kTailRegs;
  float2 pm[kTailRegs];
#pragma unroll
  for (int i = 0; i < kTailRegs; ++i) {
    const int b = t + 256 * i;
    pm[i] = in_regs && b < nb ? reinterpret_cast<const float2*>(a.part)[b] : make_float2(0.0f, 0.0f);
  }
  const int st_step = a.st && t == 0 ? a.st->step : 0;
  const int st_pos = a.st && t == 0 ? a.st->pos : 0;
  float gm = -3.402823466e38f;
  if (in_regs) {
#pragma unroll
    for (int i = 0; i < kTailRegs; ++i)
      if (t + 256 * i < nb) gm = fmaxf(gm, pm[i].x);
  } else {
    for (int b = t; b < nb; b += 256) gm = fmaxf(gm, a.part[2 * b]);
  }
  gm = wave_max(gm);
  if (lane == 0) wred[wave] = gm;
  __syncthreads();
  gm = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
  float gs = 0.0f;
  if (in_regs) {
#pragma unroll
    for (int i = 0; i < kTailRegs; ++i)
      if (t + 256 * i < nb) gs = gs + pm[i].y * es_exp(pm[i].x - gm);
  } else {
    for (int b = t; b < nb; b += 256) gs = gs + a.part[2 * b + 1] * es_exp(a.part[2 * b] - gm);
  }
  gs = tree64(gs);
  if (lane == 0) wred2[wave] = gs;
  __syncthreads();
  gs = (wred2[0] + wred2[1]) + (wred2[2] + wred2[3]);
  const float lse = rbf(es_log(gs) + gm);
  const float target = rbf(gm - lse);
  unsigned int first = 0xffffffffu;
  if (in_regs) {
#pragma unroll
    for (int i = 0; i < kTailRegs; ++i) {
      const int b = t + 256 * i;
      if (b < nb && rbf(pm[i].x - lse) == target && (unsigned int)b < first) first = (unsigned int)b;
    }
  } else {
    for (int b = t; b < nb; b += 256)
      if (rbf(a.part[2 * b] - lse) == target && (unsigned int)b < first) first = (unsigned int)b;
  }
  first = wave_umin(first);
  if (lane == 0) wmin[wave] = first;
  __syncthreads();
  first = wmin[0];
  for (int w = 1; w < 4; ++w) first = wmin[w] < first ? wmin[w] : first;
  __syncthreads();
  unsigned int best = 0xffffffffu;
  if (first < (unsigned int)nb) {
    const int r = (int)first * kRowsPerBlock + t;
    if (r < vocab && rbf(bf2f(a.logits[r]) - lse) == target) best = (unsigned int)r;
  }
  best = wave_umin(best);
  if (lane == 0) wmin[wave] = best;
  __syncthreads();
  if (t == 0) {
    unsigned int tok = wmin[0];
    for (int w = 1; w < 4; ++w) tok = wmin[w] < tok ? wmin[w] : tok;
    if (tok >= (unsigned int)vocab) tok = 0;  // unreachable unless logits are NaN
    if (a.token_out) *a.token_out = tok;
    if (a.lse_out) *a.lse_out = lse;
    if (a.st) {
      if (a.out_tokens) a.out_tokens[st_step] = tok;
      a.st->token = tok;
      a.st->step = st_step + 1;
      a.st->pos = st_pos + 1;
    }
  }
}

__global__ void k_advance(StepState* st, const uint32_t* prompt) {
  const int p = st->pos + 1;
  st->pos = p;
  st->token = prompt[p];
}

__global__ void k_set_token(StepState* st, const uint32_t* src) { st->token = *src; }

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

__device__ __forceinline__ float2 normal_pair(uint64_t seed, uint64_t i) {
  const uint64_t r = splitmix64(seed ^ (i * 0xD1B54A32D192ED03ull));
  const float u1 = ((float)(uint32_t)(r >> 40) + 0.5f) * (1.0f / 16777216.0f);
  const float u2 = ((float)(uint32_t)(r & 0xFFFFFFu)) * (1.0f / 16777216.0f);
  const float rad = sqrtf(-2.0f * logf(u1));
  return make_float2(rad * cosf(6.283185307179586f * u2), rad * sinf(6.283185307179586f * u2));
}

__global__ void k_fill_normal_bf16(uint16_t* dst, size_t n, float sigma, uint64_t seed) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; 2 * i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const float2 z = normal_pair(seed, i);
    dst[2 * i] = (uint16_t)f2bf(z.x * sigma);
    if (2 * i + 1 < n) dst[2 * i + 1] = (uint16_t)f2bf(z.y * sigma);
  }
}

__global__ void k_fill_normal_f32(float* dst, size_t n, float sigma, uint64_t seed) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; 2 * i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const float2 z = normal_pair(seed, i);
    dst[2 * i] = z.x * sigma;
    if (2 * i + 1 < n) dst[2 * i + 1] = z.y * sigma;
  }
}

// Plain streaming copy, 16 bytes per thread per step (also the reference
// point for the HBM byte counters: it reads and writes exactly `n16` x 16 B).
__global__ __launch_bounds__(256) void k_copy16(u32x4* __restrict__ dst,
                                                const u32x4* __restrict__ src, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
       i += (size_t)gridDim.x * blockDim.x)
    dst[i] = __builtin_nontemporal_load(src + i);
}

// Plain streaming read by global->LDS DMA, the fastest read pattern measured
// on this part and so the read-only ceiling beside the nameplate HBM figure:
// kReadBlocks blocks of 8 waves, each block reading one contiguous chunk in
// 8 KB steps (wave w takes the step's kilobyte w, one 16-byte DMA per lane),
// waiting after every fourth DMA of a wave until at most three are in
// flight, into an LDS ring that nothing reads. One word per block is stored
// so the launch has an output.
constexpr int kReadBlocks = 256;
typedef __attribute__((address_space(3))) void* read_lds_t;

__global__ __launch_bounds__(512) void k_read_lds(const uint8_t* __restrict__ src, size_t chunk, uint32_t* out) {
  __shared__ __attribute__((aligned(16))) uint32_t ring[8][4][256];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint8_t* p = src + (size_t)blockIdx.x * chunk + (size_t)wave * 1024 + (size_t)lane * 16;
  const size_t steps = chunk / 8192;
  for (size_t i = 0; i < steps; ++i) {
    __builtin_amdgcn_global_load_lds(p + i * 8192, (read_lds_t)&ring[wave][i & 3][0], 16, 0, kLoadNonTemporal);
    if ((i & 3) == 3) __builtin_amdgcn_s_waitcnt(3 | (7 << 4) | (15 << 8));  // vmcnt(3)
  }
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = ring[0][0][0];
}

// Block partials of launch_head_noalloc, for callers that cannot allocate:
// one copy per device, held until the process ends, shared by every such call
// on that device (calls that overlap on one device race). Each launch writes
// every partial it reads, so the array needs no clearing between calls.
constexpr int kNoAllocMaxVocab = 1 << 20;

}  // namespace

static __device__ __align__(256) float scratch[2 * ((kNoAllocMaxVocab + kRowsPerBlock - 1) / kRowsPerBlock)];

int head_noalloc_max_vocab() { return kNoAllocMaxVocab; }

// Device address of `scratch` on the current device. The host-side name of a
// __device__ array is only a handle: kernels must be given this address.
// Looked up once per device (with that device current) and kept.
static hipError_t noalloc_scratch(float** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    addr[dev] = p;
  }
  *out = static_cast<float*>(addr[dev]);
  return hipSuccess;
}

hipError_t launch_head_noalloc(HeadArgs a, hipStream_t s) {
  if (a.embed.n <= 0 || a.embed.n > kNoAllocMaxVocab) return hipErrorInvalidValue;
  float* part = nullptr;
  hipError_t e = noalloc_scratch(&part);
  if (e != hipSuccess) return e;
  a.part = part;
  return launch_head(a, s);
}

hipError_t launch_greedy(const uint16_t* logits, int count, float* part, uint32_t* token, float* lse,
                         hipStream_t s) {
  if (!logits || !part || !token || count <= 0 || count >= (1 << 22)) return hipErrorInvalidValue;
  const int nb = head_blocks(count);
  HeadArgs a{};
  a.embed.n = count;
  a.logits = const_cast<uint16_t*>(logits);  // the tail only reads them
  a.part = part;
  a.token_out = token;
  a.lse_out = lse;
  hipLaunchKernelGGL(k_logits_part, dim3(nb), dim3(256), 0, s, logits, count, part);
  hipLaunchKernelGGL(k_head_tail, dim3(1), dim3(256), 0, s, a, nb);
  return hipGetLastError();
}

size_t read_out_bytes() { return (size_t)kReadBlocks * 4; }
size_t read_granule() { return (size_t)kReadBlocks * 8192; }

hipError_t launch_read(const void* src, size_t bytes, void* out, hipStream_t s) {
  if (!src || !out || bytes == 0 || bytes % read_granule() != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_read_lds, dim3(kReadBlocks), dim3(512), 0, s, static_cast<const uint8_t*>(src),
                     bytes / kReadBlocks, static_cast<uint32_t*>(out));
  return hipGetLastError();
}

hipError_t launch_copy16(void* dst, const void* src, size_t bytes, hipStream_t s) {
  if (!dst || !src || bytes % 16 != 0) return hipErrorInvalidValue;
  if (bytes == 0) return hipSuccess;
  const size_t n16 = bytes / 16;
  size_t blocks = (n16 + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(k_copy16, dim3((unsigned)blocks), dim3(256), 0, s, static_cast<u32x4*>(dst),
                     static_cast<const u32x4*>(src), n16);
  return hipGetLastError();
}

int head_blocks(int vocab) { return (vocab + kRowsPerBlock - 1) / kRowsPerBlock; }
size_t head_scratch_bytes(int vocab) { return (size_t)head_blocks(vocab) * 2 * sizeof(float); }

hipError_t launch_head(const HeadArgs& a, hipStream_t s) {
  // vocab < 2^22 keeps every byte offset of the code table within 31 bits
  if (!a.embed.w || !a.embed.s || !a.embed.b || a.embed.k != kHidden || a.embed.n <= 0 ||
      a.embed.n >= (1 << 22) || !a.h || !a.gain || !a.logits || !a.part)
    return hipErrorInvalidValue;
  const int nb = head_blocks(a.embed.n);
  if (a.dpart)
    hipLaunchKernelGGL(k_head<true>, dim3(nb), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(k_head<false>, dim3(nb), dim3(256), 0, s, a);
  hipLaunchKernelGGL(k_head_tail, dim3(1), dim3(256), 0, s, a, nb);
  return hipGetLastError();
}

hipError_t launch_advance(StepState* st, const uint32_t* prompt, hipStream_t s) {
  if (!st || !prompt) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_advance, dim3(1), dim3(1), 0, s, st, prompt);
  return hipGetLastError();
}

hipError_t launch_set_token(StepState* st, const uint32_t* src, hipStream_t s) {
  if (!st || !src) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_set_token, dim3(1), dim3(1), 0, s, st, src);
  return hipGetLastError();
}

hipError_t launch_fill_normal_bf16(uint16_t* dst, size_t n, float sigma, uint64_t seed,
                                   hipStream_t s) {
  if (!dst) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  size_t pairs = (n + 1) / 2;
  int blocks = (int)((pairs + 255) / 256);
  if (blocks > 16384) blocks = 16384;
  hipLaunchKernelGGL(k_fill_normal_bf16, dim3(blocks), dim3(256), 0, s, dst, n, sigma, seed);
  return hipGetLastError();
}

hipError_t launch_fill_normal_f32(float* dst, size_t n, float sigma, uint64_t seed,
                                  hipStream_t s) {
  if (!dst) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  size_t pairs = (n + 1) / 2;
  int blocks = (int)((pairs + 255) / 256);
  if (blocks > 16384) blocks = 16384;
  hipLaunchKernelGGL(k_fill_normal_f32, dim3(blocks), dim3(256), 0, s, dst, n, sigma, seed);
  return hipGetLastError();
}

}  // namespace es
