// Weight blob layout and the seeded random-init generator.
#include "es_weights.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>

namespace es {

uint16_t host_f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float host_bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// attention.metal:62-63: exp2(-(pair/32) * log2(1e7)) with the exponent formed
// in fp32 as written and exp2 evaluated accurately, rounded once to fp32.
float rope_inv_freq_host(int pair) {
  const float t = -((float)pair / 32.0f) * 23.253496170043945f;
  return (float)std::exp2((double)t);
}

namespace {

struct Builder {
  std::vector<TensorDesc> t;
  uint64_t off = 0;
  void add(const std::string& name, DType dt, std::vector<int64_t> shape) {
    uint64_t n = 1;
    for (auto d : shape) n *= (uint64_t)d;
    const uint64_t bytes = n * (dt == kBF16 ? 2 : 4);
    t.push_back({name, dt, shape, off, bytes});
    off = (off + bytes + 255) & ~uint64_t(255);
  }
  void q4(const std::string& name, int n, int k) {
    add(name + ".weight", kU32, {n, k / 8});
    add(name + ".scales", kBF16, {n, k / 64});
    add(name + ".biases", kBF16, {n, k / 64});
  }
};

inline uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// Counter-based N(0,1): element i of stream `key`.
inline float normal_at(uint64_t key, uint64_t i) {
  const uint64_t r = splitmix64(key ^ splitmix64(i));
  const double u1 = ((double)(r >> 11) + 0.5) * (1.0 / 9007199254740992.0);
  const uint64_t r2 = splitmix64(r);
  const double u2 = (double)(r2 >> 11) * (1.0 / 9007199254740992.0);
  return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
}
inline float uniform_at(uint64_t key, uint64_t i) {
  const uint64_t r = splitmix64(key ^ splitmix64(i));
  return (float)(((double)(r >> 11) + 0.5) * (1.0 / 9007199254740992.0));
}

uint64_t name_key(uint64_t seed, const std::string& name) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char c : name) h = (h ^ c) * 1099511628211ull;
  return splitmix64(seed ^ h);
}

template <class F>
void parallel_rows(int rows, int threads, F f) {
  threads = std::max(1, std::min(threads, rows));
  std::vector<std::thread> pool;
  for (int t = 0; t < threads; ++t) {
    pool.emplace_back([=]() {
      const int r0 = (int)((int64_t)rows * t / threads), r1 = (int)((int64_t)rows * (t + 1) / threads);
      for (int r = r0; r < r1; ++r) f(r);
    });
  }
  for (auto& th : pool) th.join();
}

}  // namespace

std::vector<TensorDesc> weight_layout(const ModelShape& m, uint64_t* total_bytes) {
  Builder b;
  b.q4("embed_tokens", m.vocab, 1024);
  b.add("norm.weight", kBF16, {1024});
  for (int l = 0; l < m.n_layers; ++l) {
    const std::string p = "layers." + std::to_string(l);
    b.add(p + ".input_layernorm.weight", kBF16, {1024});
    b.add(p + ".post_attention_layernorm.weight", kBF16, {1024});
    b.q4(p + ".mlp.gate_proj", 3584, 1024);
    b.q4(p + ".mlp.up_proj", 3584, 1024);
    b.q4(p + ".mlp.down_proj", 1024, 3584);
    if (m.is_attention(l)) {
      const std::string a = p + ".self_attn";
      b.q4(a + ".q_proj", 4096, 1024);
      b.q4(a + ".k_proj", 512, 1024);
      b.q4(a + ".v_proj", 512, 1024);
      b.q4(a + ".o_proj", 1024, 2048);
      b.add(a + ".q_norm.weight", kBF16, {256});
      b.add(a + ".k_norm.weight", kBF16, {256});
    } else {
      const std::string g = p + ".linear_attn";
      b.q4(g + ".in_proj_qkv", 6144, 1024);
      b.q4(g + ".in_proj_z", 2048, 1024);
      b.q4(g + ".in_proj_a", 16, 1024);
      b.q4(g + ".in_proj_b", 16, 1024);
      b.q4(g + ".out_proj", 1024, 2048);
      b.add(g + ".conv1d.weight", kBF16, {6144, 4, 1});
      b.add(g + ".norm.weight", kBF16, {128});
      b.add(g + ".dt_bias", kBF16, {16});
      b.add(g + ".A_log", kF32, {16});
    }
  }
  if (total_bytes) *total_bytes = b.off;
  return b.t;
}

// Affine 4-bit, group 64: scale = (max-min)/15, bias = min, both rounded to
// bf16; q = clamp(round((w - bias)/scale), 0, 15) against the rounded pair.
void quantize_row_q4(const float* w, int k, uint32_t* codes, uint16_t* scales, uint16_t* biases) {
  for (int g = 0; g < k / 64; ++g) {
    const float* x = w + g * 64;
    float mn = x[0], mx = x[0];
    for (int i = 1; i < 64; ++i) {
      mn = std::min(mn, x[i]);
      mx = std::max(mx, x[i]);
    }
    const uint16_t sb = host_f32_to_bf16((mx - mn) / 15.0f);
    const uint16_t bb = host_f32_to_bf16(mn);
    scales[g] = sb;
    biases[g] = bb;
    const float s = host_bf16_to_f32(sb), b0 = host_bf16_to_f32(bb);
    for (int i = 0; i < 64; i += 8) {
      uint32_t word = 0;
      for (int j = 0; j < 8; ++j) {
        int q = 0;
        if (s > 0.0f) q = (int)std::lrint((x[i + j] - b0) / s);
        q = std::max(0, std::min(15, q));
        word |= (uint32_t)q << (4 * j);
      }
      codes[(g * 64 + i) / 8] = word;
    }
  }
}

bool weights_random(const ModelShape& m, uint64_t seed, void* blob, uint64_t bytes, int threads) {
  uint64_t total = 0;
  const auto layout = weight_layout(m, &total);
  if (!blob || bytes < total) return false;
  uint8_t* base = static_cast<uint8_t*>(blob);
  std::memset(base, 0, total);
  if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());
  for (size_t i = 0; i < layout.size(); ++i) {
    const TensorDesc& d = layout[i];
    const std::string& n = d.name;
    const uint64_t key = name_key(seed, n);
    const bool is_w = n.size() > 7 && n.compare(n.size() - 7, 7, ".weight") == 0;
    if (d.dtype == kU32 && is_w) {
      // Q4 triple: this .weight, then .scales and .biases
      const int rows = (int)d.shape[0], k = (int)d.shape[1] * 8;
      uint32_t* codes = reinterpret_cast<uint32_t*>(base + d.offset);
      uint16_t* sc = reinterpret_cast<uint16_t*>(base + layout[i + 1].offset);
      uint16_t* bi = reinterpret_cast<uint16_t*>(base + layout[i + 2].offset);
      parallel_rows(rows, threads, [&](int r) {
        std::vector<float> w(k);
        for (int c = 0; c < k; ++c) w[c] = 0.02f * normal_at(key, (uint64_t)r * k + c);
        quantize_row_q4(w.data(), k, codes + (size_t)r * (k / 8), sc + (size_t)r * (k / 64),
                        bi + (size_t)r * (k / 64));
      });
      i += 2;
      continue;
    }
    const uint64_t count = d.bytes / (d.dtype == kBF16 ? 2 : 4);
    if (n.find("layernorm") != std::string::npos || n == "norm.weight" ||
        n.find("q_norm") != std::string::npos || n.find("k_norm") != std::string::npos ||
        n.find("linear_attn.norm") != std::string::npos) {
      uint16_t* p = reinterpret_cast<uint16_t*>(base + d.offset);
      for (uint64_t e = 0; e < count; ++e) p[e] = host_f32_to_bf16(1.0f + 0.1f * normal_at(key, e));
    } else if (n.find("conv1d") != std::string::npos) {
      uint16_t* p = reinterpret_cast<uint16_t*>(base + d.offset);
      for (uint64_t e = 0; e < count; ++e) p[e] = host_f32_to_bf16(0.5f * normal_at(key, e));
    } else if (n.find("A_log") != std::string::npos) {
      float* p = reinterpret_cast<float*>(base + d.offset);
      for (uint64_t e = 0; e < count; ++e) p[e] = std::log(0.5f + 1.5f * uniform_at(key, e));
    } else if (n.find("dt_bias") != std::string::npos) {
      uint16_t* p = reinterpret_cast<uint16_t*>(base + d.offset);
      for (uint64_t e = 0; e < count; ++e) p[e] = host_f32_to_bf16(-1.0f + 0.5f * normal_at(key, e));
    } else {
      return false;  // every tensor must be covered above
    }
  }
  return true;
}

}  // namespace es
