// Checkpoint directory loading (config.json + *.safetensors) into the weight
// blob layout of es_weights.hpp.
#pragma once
#include <cstdint>
#include <string>

namespace es {

// config.json of an MLX Qwen3.5-0.8B checkpoint: text_config must have
// hidden_size 1024, num_hidden_layers 24 and vocab_size 248320 (weights.rs:12-15);
// otherwise "unsupported model configuration".
bool checkpoint_config(const std::string& dir, int* n_layers, int* vocab, std::string* err);

// The language_model.model.* tensors of every *.safetensors file in dir,
// validated as weights.rs:16-53 / model.rs:38-79 do, copied into blob (layout
// of weight_layout(n_layers, vocab); at least that many bytes).
bool checkpoint_load(const std::string& dir, int n_layers, int vocab, void* blob, uint64_t bytes,
                     std::string* err);

}  // namespace es
