// Host weight blob: one contiguous buffer holding every tensor of the model,
// named as in the reference checkpoint under language_model.model.*
// (model.rs:41-78, weights.rs:50-52). The same byte layout is uploaded to
// the GPU in one copy, so device tensor addresses are base + offset.
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace es {

enum DType { kU32 = 0, kBF16 = 1, kF32 = 2 };

struct TensorDesc {
  std::string name;
  DType dtype;
  std::vector<int64_t> shape;
  uint64_t offset;
  uint64_t bytes;
};

struct ModelShape {
  int n_layers;
  int vocab;
  bool is_attention(int l) const { return l % 4 == 3; }  // model.rs:51
};

// Full tensor table in blob order; offsets are 256-byte aligned.
std::vector<TensorDesc> weight_layout(const ModelShape& m, uint64_t* total_bytes);

// Seeded random-init model: Q4 matrices quantised (affine, 4-bit, group 64,
// bf16 scale/bias) from N(0, 0.02); RMSNorm gains bf16(1 + 0.1 N(0,1));
// conv1d weights bf16(N(0, 0.5)); A_log = ln U(0.5, 2); dt_bias bf16(N(-1, 0.5)).
// Deterministic for a seed, independent of the thread count.
bool weights_random(const ModelShape& m, uint64_t seed, void* blob, uint64_t bytes, int threads);

// Affine 4-bit group-64 quantisation of one row of fp32 values.
void quantize_row_q4(const float* w, int k, uint32_t* codes, uint16_t* scales, uint16_t* biases);

uint16_t host_f32_to_bf16(float f);
float host_bf16_to_f32(uint16_t b);
float rope_inv_freq_host(int pair);

}  // namespace es
