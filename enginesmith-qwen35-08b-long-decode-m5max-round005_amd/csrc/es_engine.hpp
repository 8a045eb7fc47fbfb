// Decode engine: the MI355X counterpart of the reference's Model
// (model.rs:28-180). It owns the weights, the persistent decode state (GDN
// conv rings and fp32 states, bf16 KV caches), the scratch buffers, and one
// hipGraph per step kind and attention split count. A step's position and
// token live in device memory (StepState), so the same graph replays for
// every token and the vocab head feeds its argmax to the next step's
// embedding without a host round trip.
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "es_kernels.hpp"
#include "es_weights.hpp"

namespace es {

struct LayerDev {
  bool attention;
  const uint16_t* input_norm;
  const uint16_t* post_norm;
  Q4 gate, up, down;
  // packed scale|bias<<16 group words of the XCD kernels: (gate, up)
  // interleaved, down by XCD octet; GDN qkv, z, a then b, out by head pair
  uint2* gu_sb;
  uint32_t* down_sb;
  uint32_t* qkv_sb;
  uint32_t* z_sb;
  uint32_t* ab_sb;
  uint32_t* out_sb;
  uint32_t* o_sb;  // attention o_proj by head (launch_pack_out_pairs), every engine mode
  // GDN
  Q4 qkv, z, a, b, out;
  const uint16_t* conv_w;
  const uint16_t* gdn_norm;
  const uint16_t* dt_bias;
  const float* a_log;
  uint16_t* ring;   // [4, 6144]
  float* state;     // [16, 128, 128]
  // attention
  Q4 q, k, v, o;
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  uint16_t* kcache; // [2, capacity, 256]
  uint16_t* vcache;
};

class Engine {
 public:
  static Engine* create(const void* blob, uint64_t bytes, int n_layers, int vocab, int capacity,
                        std::string* err);
  ~Engine();

  // Model::generate (model.rs:97-122). Returns 0 or an error (message in err).
  int generate(const uint32_t* prompt, int len, int count, bool reset, uint32_t* out,
               std::string* err);
  // Teacher-forced decode: step i consumes tokens[i]; argmax_out[i] is the
  // greedy pick after it. logits_out (optional, host) receives [n, vocab] bf16.
  int forced_decode(const uint32_t* tokens, int n, uint32_t* argmax_out, uint16_t* logits_out,
                    std::string* err);
  // Prompt consumption (model.rs:106-109): chunk_rows >= 2 consumes the
  // prompt as the reference's 2048-row forwards do, running the rows of full
  // forwards in batched chunks of at most chunk_rows rows (results do not
  // depend on chunk_rows); 0 replays one decode step per prompt token.
  int set_prefill(int chunk_rows, std::string* err);
  int prefill_chunk_rows() const { return prefill_rows_; }
  // How the last reset request consumed its prompt: batched chunks of
  // full-forward rows, rows of a routed last forward, decode-kernel rows.
  struct PromptSplit {
    int chunks = 0, routed_rows = 0, decode_rows = 0;
  };
  PromptSplit last_prompt_split() const { return split_; }
  void cancel() { cancelled_.store(true); }
  void clear_cancel() { cancelled_.store(false); }
  int position() const { return position_; }
  bool has_pending() const { return has_pending_; }
  uint32_t pending() const { return pending_; }

  // State handoff (host copies). which: 0 = K cache, 1 = V cache.
  int read_kv(int layer, int which, int pos0, int count, void* host, std::string* err);
  int write_kv(int layer, int which, int pos0, int count, const void* host, std::string* err);
  // ring [4,6144] bf16 and state [16,128,128] f32 of a GDN layer
  int read_gdn(int layer, void* ring_host, void* state_host, std::string* err);
  int write_gdn(int layer, const void* ring_host, const void* state_host, std::string* err);
  // Synthetic context of `length` consumed tokens: N(0,1) KV rows, N(0,0.1)
  // GDN states, N(0,1) rings; the pending token is `token`.
  int fill_synthetic(int length, uint64_t seed, uint32_t token, std::string* err);
  int set_position(int position, uint32_t pending, std::string* err);

  // Timing (HIP events on the engine stream).
  int time_decode(int steps, int warmup, double* ms_total, std::string* err);
  // which: 0 = the three attention launches, 1 = scores, 2 = chains, 3 = merge.
  int time_attention(int layer, int reps, int which, double* ms_avg, std::string* err);
  int time_head(int reps, double* ms_avg, std::string* err);

  bool fused_mlp() const { return fused_mlp_; }
  // Decode steps on the XCD-cooperative kernels (on, when the start-up probe
  // allowed them) or on one launch per dependency; both give the same bits.
  int set_xcd_kernels(bool on, std::string* err);
  // Test hook for the exchange failure path (1: set the error word; 2: move
  // one block's exchange count so waits on its words run out).
  int inject_exchange_fault(int mode, std::string* err);
  int n_layers() const { return shape_.n_layers; }
  int vocab() const { return shape_.vocab; }
  int capacity() const { return capacity_; }
  static int splits_for(int length);

 private:
  Engine() = default;
  int init(const void* blob, uint64_t bytes, std::string* err);
  void reset_state();
  hipError_t enqueue_layers(hipStream_t s, int splits);
  hipError_t enqueue_step(hipStream_t s, int splits, bool with_head);
  hipGraphExec_t graph(int kind, int splits, int steps, std::string* err);
  // Enqueue `n` steps of one kind from absolute position first_pos: whole
  // kGraphSteps-step graphs, then single-step graphs for the rest.
  std::vector<std::pair<int, int>> step_plan(int first_pos, int n) const;
  int launch_steps(int kind, int first_pos, int n, std::string* err);
  static constexpr int kGraphSteps = 16;
  int run_steps(int kind, int first_pos, int count, const uint32_t* forced_dev,
                uint16_t* logits_out, std::string* err);
  int upload_state(int pos, int step, uint32_t token, std::string* err);
  // Batched forward over prompt_[pos0 .. pos0+m) without output (encode_forward
  // with rows > 1, model.rs:228-343); m <= prefill_rows_.
  // Chunks rotate over kPrefillStreams prefill streams (slot = chunk index
  // mod kPrefillStreams); with wait_prev, each layer's state update waits for
  // the previous chunk's update of the same layer, so consecutive chunks
  // overlap one layer apart.
  // With `routed`, linears below their row limit run qmv_q4 rows (the
  // reference's last, shorter forward); otherwise every linear is a GEMM.
  int prefill_rows(int pos0, int m, int slot, bool wait_prev, bool routed, std::string* err);
  int ensure_prefill_buffers(std::string* err);
  // Consume the first n prompt tokens (host copy `prompt`, device copy
  // prompt_) in chunks or steps; the state then stands at position n.
  int consume_prompt(const uint32_t* prompt, int n, std::string* err);
  AttnArgs attn_args(const LayerDev& L, int splits);
  hipError_t launch_attention_part(const AttnArgs& a, int which);

  ModelShape shape_{};
  int capacity_ = 0;
  hipStream_t stream_ = nullptr;
  uint8_t* d_weights_ = nullptr;
  std::vector<LayerDev> layers_;
  Q4 embed_{};
  const uint16_t* final_norm_ = nullptr;
  std::vector<void*> allocations_;

  // scratch
  uint16_t* h_ = nullptr;       // residual stream [1024]
  uint16_t* z_ = nullptr;       // [2048]
  uint16_t* ab_ = nullptr;      // [32]
  uint16_t* y_ = nullptr;       // [2048] GDN readout / attention gated output
  uint16_t* q_ = nullptr;       // [4096]
  uint16_t* k_ = nullptr;       // [512]
  uint16_t* v_ = nullptr;       // [512]
  uint16_t* act_ = nullptr;     // [3584]
  uint16_t* logits_ = nullptr;  // [vocab]
  float* head_part_ = nullptr;
  void* attn_scratch_ = nullptr;  // chain outputs, chain (max, sum)
  float* proj_part_ = nullptr;    // [16, 1024] head partials of out_proj / o_proj
  uint16_t* hmid_ = nullptr;      // [1024] residual after the attention / GDN mixer
  // XCD-cooperative kernels (k_gdn_xcd for GDN layers, k_mlp_xcd for every
  // MLP), used when the start-up probe sees the blocks of a 256-block launch
  // dealt to the 8 XCDs in turn
  bool fused_mlp_ = false;
  bool xcd_ok_ = false;           // the probe's verdict (packed words exist)
  float* dpart_ = nullptr;        // [8, 1024] down-projection octet partials
  uint32_t* xact_ = nullptr;      // [8, 512] activation exchange words (value | tag << 16)
  uint32_t* xgdn_ = nullptr;      // [8, 2, 648] GDN exchange words (k_gdn_xcd)
  uint32_t* xflags_ = nullptr;    // [8, 32] per-block exchange counts
  uint32_t* err_ = nullptr;       // device error word of the cooperative kernels
  int check_device_error(std::string* err);
  int probe_placement(bool* ok, std::string* err);
  int clear_exchanges(std::string* err);
  float* inv_freq_ = nullptr;
  StepState* st_ = nullptr;
  uint32_t* prompt_ = nullptr;  // [capacity]
  uint32_t* out_ = nullptr;     // [capacity]
  uint32_t* forced_ = nullptr;  // [capacity]

  // batched prefill buffers, rows = prefill_rows_ (allocated on first use)
  static constexpr int kDefaultPrefillRows = 4096;
  static constexpr int kRefChunk = 2048;    // the reference's forward rows (model.rs:7)
  static constexpr int kMaxRowLimit = 33;   // largest qmv_q4 row limit (model.rs:191)
  int prefill_rows_ = kDefaultPrefillRows;
  int prefill_alloc_rows_ = 0;
  struct PrefillBuffers {
    uint16_t *h, *u, *raw, *z, *a, *b, *q, *k, *v, *y, *gated, *qp, *kp, *vp, *query, *o, *act;
    float *g, *beta;
  };
  static constexpr int kPrefillStreams = 2;
  PrefillBuffers pf_[kPrefillStreams]{};
  hipStream_t pstream_[kPrefillStreams] = {};
  hipEvent_t state_done_[kPrefillStreams][64] = {};  // [slot][layer]: the chunk's update of that layer's state
  hipEvent_t join_ev_[1 + kPrefillStreams] = {};

  struct GraphEntry {
    int kind;
    int splits;
    int steps;
    hipGraph_t g;
    hipGraphExec_t exec;
  };
  std::vector<GraphEntry> graphs_;

  PromptSplit split_{};
  int position_ = 0;
  bool has_pending_ = false;
  uint32_t pending_ = 0;
  std::atomic<bool> cancelled_{false};
};

}  // namespace es
