// Decode engine implementation (see es_engine.hpp).
#include "es_engine.hpp"

#include <algorithm>
#include <cstring>
#include <map>

namespace es {

namespace {

constexpr int kKindDecode = 0;  // layers + vocab head (advances via the head)
constexpr int kKindPrompt = 1;  // layers + advance (prompt consumption)

#define ES_HIP(expr, what)                                                 \
  do {                                                                     \
    hipError_t e_ = (expr);                                                \
    if (e_ != hipSuccess) {                                                \
      if (err) *err = std::string(what) + ": " + hipGetErrorString(e_);    \
      return 2;                                                            \
    }                                                                      \
  } while (0)

}  // namespace

// The attention launch shape does not depend on the length, so one graph
// serves every step; the value is the `blocks` the launch arguments carry.
int Engine::splits_for(int length) {
  (void)length;
  return 64;
}

Engine* Engine::create(const void* blob, uint64_t bytes, int n_layers, int vocab, int capacity,
                       std::string* err) {
  if (n_layers < 1 || n_layers > 64 || vocab < 1 || vocab > (1 << 24) || capacity < 4 ||
      capacity > (1 << 22)) {
    if (err) *err = "invalid engine configuration";
    return nullptr;
  }
  Engine* e = new Engine();
  e->shape_ = {n_layers, vocab};
  e->capacity_ = capacity;
  if (e->init(blob, bytes, err) != 0) {
    delete e;
    return nullptr;
  }
  return e;
}

Engine::~Engine() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (hipStream_t ps : pstream_)
    if (ps) {
      (void)hipStreamSynchronize(ps);
      (void)hipStreamDestroy(ps);
    }
  for (auto& row : state_done_)
    for (hipEvent_t e : row)
      if (e) (void)hipEventDestroy(e);
  for (hipEvent_t e : join_ev_)
    if (e) (void)hipEventDestroy(e);
  for (auto& g : graphs_) {
    (void)hipGraphExecDestroy(g.exec);
    (void)hipGraphDestroy(g.g);
  }
  for (void* p : allocations_) (void)hipFree(p);
  if (stream_) (void)hipStreamDestroy(stream_);
}

int Engine::init(const void* blob, uint64_t bytes, std::string* err) {
  uint64_t total = 0;
  const auto layout = weight_layout(shape_, &total);
  if (!blob || bytes < total) {
    if (err) *err = "weight blob too small for the model shape";
    return 1;
  }
  ES_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
  auto alloc = [&](size_t n) -> void* {
    void* p = nullptr;
    if (hipMalloc(&p, std::max<size_t>(n, 256)) != hipSuccess) return nullptr;
    allocations_.push_back(p);
    return p;
  };
  d_weights_ = static_cast<uint8_t*>(alloc(total));
  if (!d_weights_) {
    if (err) *err = "device allocation of weights failed";
    return 2;
  }
  ES_HIP(hipMemcpy(d_weights_, blob, total, hipMemcpyHostToDevice), "weight upload");

  std::map<std::string, const TensorDesc*> by_name;
  for (const auto& d : layout) by_name[d.name] = &d;
  auto ptr = [&](const std::string& n) -> void* { return d_weights_ + by_name.at(n)->offset; };
  auto q4 = [&](const std::string& n, int rows, int k) {
    return Q4{static_cast<const uint32_t*>(ptr(n + ".weight")),
              static_cast<const uint16_t*>(ptr(n + ".scales")),
              static_cast<const uint16_t*>(ptr(n + ".biases")), rows, k};
  };
  embed_ = q4("embed_tokens", shape_.vocab, 1024);
  final_norm_ = static_cast<const uint16_t*>(ptr("norm.weight"));
  layers_.resize(shape_.n_layers);
  for (int l = 0; l < shape_.n_layers; ++l) {
    LayerDev& L = layers_[l];
    const std::string p = "layers." + std::to_string(l);
    L.attention = shape_.is_attention(l);
    L.input_norm = static_cast<const uint16_t*>(ptr(p + ".input_layernorm.weight"));
    L.post_norm = static_cast<const uint16_t*>(ptr(p + ".post_attention_layernorm.weight"));
    L.gate = q4(p + ".mlp.gate_proj", 3584, 1024);
    L.up = q4(p + ".mlp.up_proj", 3584, 1024);
    L.down = q4(p + ".mlp.down_proj", 1024, 3584);
    if (L.attention) {
      const std::string a = p + ".self_attn";
      L.q = q4(a + ".q_proj", 4096, 1024);
      L.k = q4(a + ".k_proj", 512, 1024);
      L.v = q4(a + ".v_proj", 512, 1024);
      L.o = q4(a + ".o_proj", 1024, 2048);
      L.q_norm = static_cast<const uint16_t*>(ptr(a + ".q_norm.weight"));
      L.k_norm = static_cast<const uint16_t*>(ptr(a + ".k_norm.weight"));
      const size_t cache = (size_t)2 * capacity_ * 256 * sizeof(uint16_t);
      L.kcache = static_cast<uint16_t*>(alloc(cache));
      L.vcache = static_cast<uint16_t*>(alloc(cache));
      if (!L.kcache || !L.vcache) {
        if (err) *err = "device allocation of KV caches failed";
        return 2;
      }
    } else {
      const std::string g = p + ".linear_attn";
      L.qkv = q4(g + ".in_proj_qkv", 6144, 1024);
      L.z = q4(g + ".in_proj_z", 2048, 1024);
      L.a = q4(g + ".in_proj_a", 16, 1024);
      L.b = q4(g + ".in_proj_b", 16, 1024);
      L.out = q4(g + ".out_proj", 1024, 2048);
      L.conv_w = static_cast<const uint16_t*>(ptr(g + ".conv1d.weight"));
      L.gdn_norm = static_cast<const uint16_t*>(ptr(g + ".norm.weight"));
      L.dt_bias = static_cast<const uint16_t*>(ptr(g + ".dt_bias"));
      L.a_log = static_cast<const float*>(ptr(g + ".A_log"));
      L.ring = static_cast<uint16_t*>(alloc((size_t)4 * kConv * sizeof(uint16_t)));
      L.state = static_cast<float*>(alloc((size_t)16 * 128 * 128 * sizeof(float)));
      if (!L.ring || !L.state) {
        if (err) *err = "device allocation of GDN state failed";
        return 2;
      }
    }
  }
  h_ = static_cast<uint16_t*>(alloc(1024 * 2));
  z_ = static_cast<uint16_t*>(alloc(2048 * 2));
  ab_ = static_cast<uint16_t*>(alloc(32 * 2));
  y_ = static_cast<uint16_t*>(alloc(2048 * 2));
  q_ = static_cast<uint16_t*>(alloc(4096 * 2));
  k_ = static_cast<uint16_t*>(alloc(512 * 2));
  v_ = static_cast<uint16_t*>(alloc(512 * 2));
  act_ = static_cast<uint16_t*>(alloc(3584 * 2));
  logits_ = static_cast<uint16_t*>(alloc((size_t)shape_.vocab * 2));
  head_part_ = static_cast<float*>(alloc((size_t)head_blocks(shape_.vocab) * 2 * sizeof(float)));
  attn_scratch_ = alloc(attn_scratch_bytes(capacity_));
  proj_part_ = static_cast<float*>(alloc((size_t)kGdnHeads * kHidden * sizeof(float)));
  hmid_ = static_cast<uint16_t*>(alloc(1024 * 2));
  dpart_ = static_cast<float*>(alloc(8 * 1024 * sizeof(float)));
  xact_ = static_cast<uint32_t*>(alloc(8 * 512 * 4));
  xgdn_ = static_cast<uint32_t*>(alloc(8 * 2 * 648 * 4));
  xflags_ = static_cast<uint32_t*>(alloc(8 * 32 * sizeof(uint32_t)));
  err_ = static_cast<uint32_t*>(alloc(256 * sizeof(uint32_t)));
  inv_freq_ = static_cast<float*>(alloc(32 * sizeof(float)));
  st_ = static_cast<StepState*>(alloc(sizeof(StepState)));
  prompt_ = static_cast<uint32_t*>(alloc((size_t)capacity_ * 4));
  out_ = static_cast<uint32_t*>(alloc((size_t)capacity_ * 4));
  forced_ = static_cast<uint32_t*>(alloc((size_t)capacity_ * 4));
  for (void* p : {(void*)h_, (void*)z_, (void*)ab_, (void*)y_, (void*)q_, (void*)k_, (void*)v_,
                  (void*)act_, (void*)logits_, (void*)head_part_,
                  attn_scratch_, (void*)proj_part_, (void*)hmid_, (void*)dpart_, (void*)xact_, (void*)xgdn_,
                  (void*)xflags_, (void*)err_, (void*)inv_freq_, (void*)st_,
                  (void*)prompt_,
                  (void*)out_, (void*)forced_}) {
    if (!p) {
      if (err) *err = "device allocation of scratch failed";
      return 2;
    }
  }
  float inv_freq[32];
  for (int i = 0; i < 32; ++i) inv_freq[i] = rope_inv_freq_host(i);
  ES_HIP(hipMemcpy(inv_freq_, inv_freq, sizeof(inv_freq), hipMemcpyHostToDevice), "inv_freq");
  // Clears go on the engine stream: a null-stream memset is asynchronous and
  // not ordered with this non-blocking stream, so a late one could zero K/V
  // rows the first steps have already written.
  ES_HIP(hipMemsetAsync(h_, 0, 1024 * 2, stream_), "memset");
  for (auto& L : layers_)
    if (L.attention) {
      const size_t cache = (size_t)2 * capacity_ * 256 * sizeof(uint16_t);
      ES_HIP(hipMemsetAsync(L.kcache, 0, cache, stream_), "memset kv");
      ES_HIP(hipMemsetAsync(L.vcache, 0, cache, stream_), "memset kv");
    }
  reset_state();
  if (int rc = probe_placement(&xcd_ok_, err)) return rc;
  fused_mlp_ = xcd_ok_;
  for (auto& L : layers_) {
    if (!L.attention) continue;
    L.o_sb = static_cast<uint32_t*>(alloc((size_t)8 * 1024 * 4 * 4));
    if (!L.o_sb) {
      if (err) *err = "device allocation of packed group words failed";
      return 2;
    }
    ES_HIP(launch_pack_out_pairs(L.o.s, L.o.b, L.o_sb, stream_), "pack");
  }
  if (fused_mlp_) {
    // the XCD kernels read each Q4 group's scale and bias as one word
    for (auto& L : layers_) {
      const size_t ffn_groups = (size_t)3584 * 16;
      L.gu_sb = static_cast<uint2*>(alloc(ffn_groups * sizeof(uint2)));
      L.down_sb = static_cast<uint32_t*>(alloc((size_t)8 * 1024 * 8 * 4));
      if (!L.gu_sb || !L.down_sb) {
        if (err) *err = "device allocation of packed group words failed";
        return 2;
      }
      ES_HIP(launch_pack_sb2(L.gate.s, L.gate.b, L.up.s, L.up.b, L.gu_sb, ffn_groups, stream_), "pack");
      ES_HIP(launch_pack_down_octets(L.down.s, L.down.b, L.down_sb, stream_), "pack");
      if (L.attention) continue;
      L.qkv_sb = static_cast<uint32_t*>(alloc((size_t)kConv * 16 * 4));
      L.z_sb = static_cast<uint32_t*>(alloc((size_t)2048 * 16 * 4));
      L.ab_sb = static_cast<uint32_t*>(alloc((size_t)2 * kGdnHeads * 16 * 4));
      L.out_sb = static_cast<uint32_t*>(alloc((size_t)8 * 1024 * 4 * 4));
      if (!L.qkv_sb || !L.z_sb || !L.ab_sb || !L.out_sb) {
        if (err) *err = "device allocation of packed group words failed";
        return 2;
      }
      ES_HIP(launch_pack_sb(L.qkv.s, L.qkv.b, L.qkv_sb, (size_t)kConv * 16, stream_), "pack");
      ES_HIP(launch_pack_sb(L.z.s, L.z.b, L.z_sb, (size_t)2048 * 16, stream_), "pack");
      ES_HIP(launch_pack_sb(L.a.s, L.a.b, L.ab_sb, (size_t)kGdnHeads * 16, stream_), "pack");
      ES_HIP(launch_pack_sb(L.b.s, L.b.b, L.ab_sb + kGdnHeads * 16, (size_t)kGdnHeads * 16, stream_), "pack");
      ES_HIP(launch_pack_out_pairs(L.out.s, L.out.b, L.out_sb, stream_), "pack");
    }
  }
  return clear_exchanges(err);
}

// Placement probe for the XCD-cooperative kernels: the blocks of a 256-block
// launch must be dealt to the 8 XCDs in turn (from any start), 32 to each
// (err_ doubles as the probe's output; clear_exchanges clears it after).
int Engine::probe_placement(bool* ok, std::string* err) {
  ES_HIP(launch_xcc_probe(err_, stream_), "placement probe");
  uint32_t xcc[256];
  ES_HIP(hipMemcpyAsync(xcc, err_, sizeof(xcc), hipMemcpyDeviceToHost, stream_), "placement probe");
  ES_HIP(hipStreamSynchronize(stream_), "placement probe");
  bool good = xcc[0] < 8;
  for (int b = 0; b < 256; ++b) good = good && xcc[b] == (xcc[0] + (uint32_t)b) % 8;
  *ok = good;
  return 0;
}

// The error word, the per-block exchange counts and every exchange word back
// to zero (tag 0 on every word: the first tag a launch waits for is 1).
int Engine::clear_exchanges(std::string* err) {
  ES_HIP(hipMemsetAsync(err_, 0, 256 * sizeof(uint32_t), stream_), "memset");
  ES_HIP(hipMemsetAsync(xflags_, 0, 8 * 32 * sizeof(uint32_t), stream_), "memset");
  ES_HIP(hipMemsetAsync(xact_, 0, 8 * 512 * 4, stream_), "memset");
  ES_HIP(hipMemsetAsync(xgdn_, 0, 8 * 2 * 648 * 4, stream_), "memset");
  ES_HIP(hipStreamSynchronize(stream_), "exchange clear");
  return 0;
}

// The cooperative kernels report an exhausted exchange wait in err_ (every
// later wait then gives up at once); the batch's results are not to be
// trusted. The exchange state is cleared so the next request starts afresh,
// and the placement probe runs again: if the blocks are no longer dealt to
// the XCDs in turn, later steps run on one launch per dependency.
int Engine::check_device_error(std::string* err) {
  if (!fused_mlp_) return 0;
  uint32_t e = 0;
  ES_HIP(hipMemcpyAsync(&e, err_, sizeof(e), hipMemcpyDeviceToHost, stream_), "error word");
  ES_HIP(hipStreamSynchronize(stream_), "error word");
  if (e == 0) return 0;
  bool ok = false;
  if (int rc = probe_placement(&ok, err)) return rc;
  if (int rc = clear_exchanges(err)) return rc;
  if (!ok) {
    std::string ignored;
    (void)set_xcd_kernels(false, &ignored);
    xcd_ok_ = false;
  }
  if (err) *err = "decode kernels: an XCD exchange wait timed out";
  return 2;
}

// Test hook: mode 1 sets the error word (every wait of the next launches
// gives up at once); mode 2 moves block 0's exchange count away from its
// XCD's, so the waits on its words run to their spin limit.
int Engine::inject_exchange_fault(int mode, std::string* err) {
  if (!fused_mlp_) {
    if (err) *err = "the XCD-cooperative kernels are off";
    return 1;
  }
  if (mode == 1) {
    const uint32_t v = 2u;
    ES_HIP(hipMemcpyAsync(err_, &v, sizeof(v), hipMemcpyHostToDevice, stream_), "fault");
  } else if (mode == 2) {
    uint32_t c = 0;
    ES_HIP(hipMemcpyAsync(&c, xflags_, sizeof(c), hipMemcpyDeviceToHost, stream_), "fault");
    ES_HIP(hipStreamSynchronize(stream_), "fault");
    c += 0x8000u;
    ES_HIP(hipMemcpyAsync(xflags_, &c, sizeof(c), hipMemcpyHostToDevice, stream_), "fault");
  } else {
    if (err) *err = "fault mode must be 1 or 2";
    return 1;
  }
  ES_HIP(hipStreamSynchronize(stream_), "fault");
  return 0;
}

// model.rs:93-96: position 0, no pending token, zeroed GDN history and state.
void Engine::reset_state() {
  position_ = 0;
  has_pending_ = false;
  pending_ = 0;
  for (auto& L : layers_)
    if (!L.attention) {
      (void)hipMemsetAsync(L.ring, 0, (size_t)4 * kConv * 2, stream_);
      (void)hipMemsetAsync(L.state, 0, (size_t)16 * 128 * 128 * 4, stream_);
    }
}

AttnArgs Engine::attn_args(const LayerDev& L, int splits) {
  AttnArgs a{};
  a.q_proj = q_;
  a.k_proj = k_;
  a.v_proj = v_;
  a.q_gain = L.q_norm;
  a.k_gain = L.k_norm;
  a.kcache = L.kcache;
  a.vcache = L.vcache;
  a.capacity = capacity_;
  a.inv_freq = inv_freq_;
  attn_bind_scratch(a, attn_scratch_);
  a.blocks = splits;
  a.gated = y_;
  a.query_out = nullptr;
  a.st = st_;
  a.pos_val = 0;
  return a;
}

// Kernel order of encode_forward with rows == 1 (model.rs:228-307), per
// layer: GDN = input norm + projections, recurrence + gated norm + out_proj
// head partials, residual + post norm + gate/up, down + residual (4
// launches); attention = input norm + q/k/v, fused attention, merge + gate +
// o_proj head partials, residual + post norm + gate/up, down + residual (5).
// The embedding is fused into layer 0's first launch.
hipError_t Engine::enqueue_layers(hipStream_t s, int splits) {
  hipError_t e;
  for (int l = 0; l < shape_.n_layers; ++l) {
    const LayerDev& L = layers_[l];
    NormMultiArgs nm{};
    nm.x = h_;
    nm.gain = L.input_norm;
    nm.st = st_;
    if (l == 0) {
      nm.embed = embed_;
      nm.h_out = h_;
    } else if (fused_mlp_) {
      // the previous layer's MLP left the stream after its mixer and the down
      // projection's octet partials: their sum is this layer's input
      nm.x = hmid_;
      nm.dpart = dpart_;
      nm.h_out = h_;
    }
    auto mlp = [&](int nparts) -> hipError_t {
      if (fused_mlp_) {
        MlpXcdArgs m{};
        m.gate = L.gate;
        m.up = L.up;
        m.down = L.down;
        m.gu_sb = L.gu_sb;
        m.down_sb = L.down_sb;
        m.h_old = h_;
        m.part = proj_part_;
        m.h_mid = hmid_;
        m.gain = L.post_norm;
        m.dpart = dpart_;
        m.xact = xact_;
        m.flags = xflags_;
        m.err = err_;
        return launch_mlp_xcd(m, nparts, s);
      }
      hipError_t r = launch_norm_gate_up_parts(L.gate, L.up, h_, proj_part_, nparts, hmid_, L.post_norm, act_, s);
      if (r != hipSuccess) return r;
      // MLP down projection; its residual is the stream after the mixer (hmid_)
      return launch_qmv(L.down, act_, hmid_, h_, nullptr, s);
    };
    if (!L.attention && fused_mlp_) {
      // the whole GDN mixer up to its out_proj head partials in one launch
      GdnXcdArgs g{};
      if (l == 0) {
        g.embed = embed_;
      } else {
        g.x = hmid_;
        g.dpart = dpart_;
      }
      g.h_out = h_;
      g.gain = L.input_norm;
      g.qkv = L.qkv;
      g.z = L.z;
      g.a = L.a;
      g.b = L.b;
      g.out = L.out;
      g.qkv_sb = L.qkv_sb;
      g.z_sb = L.z_sb;
      g.ab_sb = L.ab_sb;
      g.out_sb = L.out_sb;
      g.conv_w = L.conv_w;
      g.norm_w = L.gdn_norm;
      g.dt_bias = L.dt_bias;
      g.a_log = L.a_log;
      g.ring = L.ring;
      g.state = L.state;
      g.part = proj_part_;
      g.xbuf = xgdn_;
      g.flags = xflags_;
      g.err = err_;
      g.st = st_;
      if ((e = launch_gdn_xcd(g, s)) != hipSuccess) return e;
      if ((e = mlp(8)) != hipSuccess) return e;  // the eight head-pair partials
    } else if (!L.attention) {
      nm.count = 4;
      nm.m[0] = L.qkv; nm.y[0] = L.ring;
      nm.m[1] = L.z;   nm.y[1] = z_;
      nm.m[2] = L.a;   nm.y[2] = ab_;
      nm.m[3] = L.b;   nm.y[3] = ab_ + 16;
      nm.ring0 = 1;
      if ((e = launch_norm_multi(nm, s)) != hipSuccess) return e;
      GdnRecurArgs g{};
      g.ring = L.ring;
      g.conv_w = L.conv_w;
      g.ab = ab_;
      g.a_log = L.a_log;
      g.dt_bias = L.dt_bias;
      g.state = L.state;
      g.st = st_;
      GdnOutArgs go{};
      go.r = g;
      go.z = z_;
      go.norm_w = L.gdn_norm;
      go.out = L.out;
      go.part = proj_part_;
      if ((e = launch_gdn_recur_out(go, s)) != hipSuccess) return e;
      if ((e = mlp(kGdnHeads)) != hipSuccess) return e;
    } else {
      nm.count = 3;
      nm.m[0] = L.q; nm.y[0] = q_;
      nm.m[1] = L.k; nm.y[1] = k_;
      nm.m[2] = L.v; nm.y[2] = v_;
      if ((e = launch_norm_multi(nm, s)) != hipSuccess) return e;
      const AttnArgs a = attn_args(L, splits);
      if ((e = launch_attn_fused(a, s)) != hipSuccess) return e;
      if ((e = launch_attn_merge_out(a, L.o, L.o_sb, proj_part_, s)) != hipSuccess) return e;
      if ((e = mlp(kQHeads)) != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

hipError_t Engine::enqueue_step(hipStream_t s, int splits, bool with_head) {
  hipError_t e = enqueue_layers(s, splits);
  if (e != hipSuccess) return e;
  if (with_head) {
    HeadArgs h{};
    h.embed = embed_;
    h.h = h_;
    if (fused_mlp_) {
      h.h = hmid_;
      h.dpart = dpart_;
    }
    h.gain = final_norm_;
    h.logits = logits_;
    h.part = head_part_;
    h.st = st_;
    h.out_tokens = out_;
    return launch_head(h, s);
  }
  return launch_advance(st_, prompt_, s);
}

// A graph holds `steps` consecutive steps of one kind. Every step reads its
// position and token from the device-side step state and advances it, so the
// same graph serves any starting position. Within one graph the steps follow
// each other as ordinary kernel boundaries; between graph launches the runtime
// adds a gap of about 9 us and the first kernel starts with cold caches.
hipGraphExec_t Engine::graph(int kind, int splits, int steps, std::string* err) {
  for (auto& g : graphs_)
    if (g.kind == kind && g.splits == splits && g.steps == steps) return g.exec;
  GraphEntry ge{kind, splits, steps, nullptr, nullptr};
  if (hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    if (err) *err = "hipStreamBeginCapture failed";
    return nullptr;
  }
  hipError_t qe = hipSuccess;
  for (int i = 0; i < steps && qe == hipSuccess; ++i)
    qe = enqueue_step(stream_, splits, kind == kKindDecode);
  const hipError_t ce = hipStreamEndCapture(stream_, &ge.g);
  if (qe != hipSuccess || ce != hipSuccess) {
    if (err) *err = std::string("graph capture failed: ") + hipGetErrorString(qe != hipSuccess ? qe : ce);
    if (ge.g) (void)hipGraphDestroy(ge.g);
    return nullptr;
  }
  if (hipGraphInstantiate(&ge.exec, ge.g, nullptr, nullptr, 0) != hipSuccess) {
    if (err) *err = "hipGraphInstantiate failed";
    (void)hipGraphDestroy(ge.g);
    return nullptr;
  }
  graphs_.push_back(ge);
  return ge.exec;
}

int Engine::upload_state(int pos, int step, uint32_t token, std::string* err) {
  StepState hs{pos, step, token, 0u};
  ES_HIP(hipMemcpyAsync(st_, &hs, sizeof(hs), hipMemcpyHostToDevice, stream_), "state upload");
  ES_HIP(hipStreamSynchronize(stream_), "state upload sync");
  return 0;
}

// Graph chunks of a run of n steps from first_pos: up to kGraphSteps steps
// each, every chunk on one attention route (the route changes once, at 1024
// attended positions), a remainder as one graph of its own length.
std::vector<std::pair<int, int>> Engine::step_plan(int first_pos, int n) const {
  std::vector<std::pair<int, int>> plan;  // (splits, steps)
  int done = 0;
  while (done < n) {
    const int pos = first_pos + done;
    const int splits = splits_for(pos + 1);
    int steps = std::min(kGraphSteps, n - done);
    while (steps > 1 && splits_for(pos + steps) != splits) --steps;
    plan.emplace_back(splits, steps);
    done += steps;
  }
  return plan;
}

int Engine::launch_steps(int kind, int first_pos, int n, std::string* err) {
  for (const auto& [splits, steps] : step_plan(first_pos, n)) {
    hipGraphExec_t ex = graph(kind, splits, steps, err);
    if (!ex) return 2;
    ES_HIP(hipGraphLaunch(ex, stream_), "hipGraphLaunch");
  }
  return 0;
}

// Launch `count` steps of one kind starting at absolute position first_pos.
// At most kAhead steps are in flight between cancellation checks
// (model.rs:127-139 keeps 16 outstanding). Forced tokens and per-step logits
// need host work between steps, so those runs launch one graph per step.
int Engine::run_steps(int kind, int first_pos, int count, const uint32_t* forced_dev,
                      uint16_t* logits_out, std::string* err) {
  constexpr int kAhead = 16;
  int launched = 0;
  while (launched < count) {
    if (cancelled_.load()) {
      (void)hipStreamSynchronize(stream_);
      if (err) *err = "input disconnected";
      return 3;
    }
    const int batch = std::min(kAhead, count - launched);
    if (!forced_dev && !logits_out) {
      if (int rc = launch_steps(kind, first_pos + launched, batch, err)) return rc;
      launched += batch;
      ES_HIP(hipStreamSynchronize(stream_), "step sync");
      if (int rc = check_device_error(err)) return rc;
      continue;
    }
    for (int i = 0; i < batch; ++i) {
      const int pos = first_pos + launched + i;
      hipGraphExec_t ex = graph(kind, splits_for(pos + 1), 1, err);
      if (!ex) return 2;
      if (forced_dev) {
        ES_HIP(launch_set_token(st_, forced_dev + launched + i, stream_), "set token");
      }
      ES_HIP(hipGraphLaunch(ex, stream_), "hipGraphLaunch");
      if (logits_out) {
        ES_HIP(hipMemcpyAsync(logits_out + (size_t)(launched + i) * shape_.vocab, logits_,
                              (size_t)shape_.vocab * 2, hipMemcpyDeviceToHost, stream_),
               "logits copy");
        ES_HIP(hipStreamSynchronize(stream_), "logits sync");
      }
    }
    launched += batch;
    ES_HIP(hipStreamSynchronize(stream_), "step sync");
    if (int rc = check_device_error(err)) return rc;
  }
  return 0;
}

int Engine::generate(const uint32_t* prompt, int len, int count, bool reset, uint32_t* out,
                     std::string* err) {
  if (count <= 0 || count > capacity_) {
    if (err) *err = "invalid output length";
    return 1;
  }
  int first;
  if (reset) {
    if (len <= 0 || !prompt) {
      if (err) *err = "reset needs nonempty prompt";
      return 1;
    }
    if ((int64_t)len + count - 1 > capacity_) {
      if (err) *err = "context capacity exceeded";
      return 1;
    }
    for (int i = 0; i < len; ++i)
      if (prompt[i] >= (uint32_t)shape_.vocab) {
        if (err) *err = "token outside vocabulary";
        return 1;
      }
    reset_state();
    ES_HIP(hipMemcpyAsync(prompt_, prompt, (size_t)len * 4, hipMemcpyHostToDevice, stream_),
           "prompt upload");
    if (int rc = consume_prompt(prompt, len - 1, err)) {
      reset_state();
      return rc;
    }
    position_ = len - 1;
    first = position_;
    // the first decode step consumes prompt[len-1]
    if (int rc = upload_state(position_, 0, prompt[len - 1], err)) return rc;
  } else {
    if (len != 0) {
      if (err) *err = "continuation prompt must be empty";
      return 1;
    }
    if ((int64_t)position_ + count > capacity_) {
      if (err) *err = "context capacity exceeded";
      return 1;
    }
    if (!has_pending_) {
      if (err) *err = "no continuation state";
      return 1;
    }
    if (int rc = upload_state(position_, 0, pending_, err)) return rc;
    first = position_;
  }
  if (int rc = run_steps(kKindDecode, first, count, nullptr, nullptr, err)) {
    reset_state();
    return rc;
  }
  ES_HIP(hipMemcpy(out, out_, (size_t)count * 4, hipMemcpyDeviceToHost), "token readback");
  position_ = first + count;
  pending_ = out[count - 1];
  has_pending_ = true;
  return 0;
}

int Engine::set_prefill(int chunk_rows, std::string* err) {
  // rows x 6144 element counts of the chunk buffers stay below 2^31
  if (chunk_rows < 0 || chunk_rows == 1 || chunk_rows > 65536) {
    if (err) *err = "prefill chunk rows must be 0 or 2 .. 65536";
    return 1;
  }
  prefill_rows_ = chunk_rows;
  return 0;
}

int Engine::set_xcd_kernels(bool on, std::string* err) {
  if (on && !xcd_ok_) {
    if (err) *err = "XCD-cooperative kernels unavailable: workgroups are not dealt to the XCDs in turn";
    return 1;
  }
  if (on == fused_mlp_) return 0;
  // the cached graphs hold the other kernels; every step starts from the
  // embedding, so the switch needs no state conversion
  ES_HIP(hipStreamSynchronize(stream_), "sync");
  for (auto& g : graphs_) {
    (void)hipGraphExecDestroy(g.exec);
    (void)hipGraphDestroy(g.g);
  }
  graphs_.clear();
  fused_mlp_ = on;
  return 0;
}

int Engine::ensure_prefill_buffers(std::string* err) {
  // chunks of prefill_rows_ and a routed last forward of fewer than
  // kMaxRowLimit rows
  const int rows = std::min(std::max(prefill_rows_, kMaxRowLimit), capacity_);
  if (prefill_alloc_rows_ >= rows) return 0;
  // buffers are kept until the engine is destroyed; a larger chunk size adds a
  // second, larger set
  const size_t r = (size_t)rows;
  auto alloc = [&](size_t n) -> void* {
    void* p = nullptr;
    if (hipMalloc(&p, std::max<size_t>(n, 256)) != hipSuccess) return nullptr;
    allocations_.push_back(p);
    return p;
  };
  if (!pstream_[0]) {
    for (auto& ps : pstream_) ES_HIP(hipStreamCreateWithFlags(&ps, hipStreamNonBlocking), "prefill stream");
    for (int slot = 0; slot < kPrefillStreams; ++slot)
      for (int l = 0; l < shape_.n_layers; ++l)
        ES_HIP(hipEventCreateWithFlags(&state_done_[slot][l], hipEventDisableTiming), "prefill event");
    for (auto& e : join_ev_) ES_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming), "prefill event");
  }
  for (int slot = 0; slot < kPrefillStreams; ++slot) {
    PrefillBuffers b{};
    uint16_t** bf[] = {&b.h, &b.u, &b.raw, &b.z, &b.a, &b.b, &b.q, &b.k, &b.v, &b.y, &b.gated, &b.qp, &b.kp,
                       &b.vp, &b.query, &b.o, &b.act};
    const size_t width[] = {1024, 1024, 6144, 2048, 16, 16, 2048, 2048, 2048, 2048, 2048, 4096, 512,
                            512, 2048, 2048, 3584};
    for (size_t i = 0; i < sizeof(width) / sizeof(width[0]); ++i) {
      *bf[i] = static_cast<uint16_t*>(alloc(r * width[i] * 2));
      if (!*bf[i]) {
        if (err) *err = "device allocation of prefill buffers failed";
        return 2;
      }
    }
    b.g = static_cast<float*>(alloc(r * 16 * 4));
    b.beta = static_cast<float*>(alloc(r * 16 * 4));
    if (!b.g || !b.beta) {
      if (err) *err = "device allocation of prefill buffers failed";
      return 2;
    }
    pf_[slot] = b;
  }
  prefill_alloc_rows_ = rows;
  return 0;
}

// encode_forward with rows > 1 and no output (model.rs:228-343): embedding
// rows; per layer input RMSNorm rows, the layer's row-batched Q4 linears,
// the mixer (GDN: conv/prepare + ring, recurrence over the rows in order,
// gated norm; attention: q/k norm + RoPE with the K/V rows written to the
// cache, causal flash attention, output gate), the output linear with the
// residual add, post RMSNorm rows, gate/up linears, SwiGLU, down linear with
// the residual add.
// A linear over m token rows. With `routed` (the reference's last, shorter
// forward) it takes qmv_q4 rows below the shape's row limit, as Model::linear
// does (model.rs:189-198); otherwise the GEMM (qmm_q4_nax), as for every row
// of a full 2048-row forward.
static hipError_t linear_rows(const Q4& w, const uint16_t* x, int m, bool routed,
                              const uint16_t* residual, uint16_t* y, hipStream_t s) {
  if (routed && m < qmv_row_limit(w.n, w.k)) return launch_qmv_rows(w, x, m, residual, y, nullptr, s);
  return launch_q4_gemm(w, x, m, residual, y, s);
}

int Engine::prefill_rows(int pos0, int m, int slot, bool wait_prev, bool routed, std::string* err) {
  const PrefillBuffers& b = pf_[slot];
  hipStream_t s = pstream_[slot];
  ES_HIP(launch_embed_rows(embed_, prompt_ + pos0, m, b.h, s), "prefill embedding");
  for (int l = 0; l < shape_.n_layers; ++l) {
    const LayerDev& L = layers_[l];
    ES_HIP(launch_rmsnorm_rows(b.h, L.input_norm, m, b.u, s), "prefill input norm");
    // the previous chunk must have finished this layer's conv ring, state or
    // K/V rows before this chunk's mixer reads them
    if (wait_prev)
      ES_HIP(hipStreamWaitEvent(s, state_done_[(slot + kPrefillStreams - 1) % kPrefillStreams][l], 0),
             "prefill wait");
    if (!L.attention) {
      if (routed) {
        ES_HIP(linear_rows(L.qkv, b.u, m, routed, nullptr, b.raw, s), "prefill qkv");
        ES_HIP(linear_rows(L.z, b.u, m, routed, nullptr, b.z, s), "prefill z");
        ES_HIP(linear_rows(L.a, b.u, m, routed, nullptr, b.a, s), "prefill a");
        ES_HIP(linear_rows(L.b, b.u, m, routed, nullptr, b.b, s), "prefill b");
      } else {
        // the four input linears share their input: one GEMM over the
        // stacked rows, each segment to its own output (the same bits)
        const Q4 w[4] = {L.qkv, L.z, L.a, L.b};
        uint16_t* const y[4] = {b.raw, b.z, b.a, b.b};
        ES_HIP(launch_q4_gemm_stacked(w, y, 4, b.u, m, s), "prefill qkv|z|a|b");
      }
      GdnPrepRowsArgs g{b.raw, L.ring, L.conv_w, b.a, b.b, L.a_log, L.dt_bias, pos0, m,
                        b.q, b.k, b.v, b.g, b.beta};
      ES_HIP(launch_gdn_prep_rows(g, s), "prefill gdn prepare");
      ES_HIP(launch_gdn_recur_rows(b.q, b.k, b.v, b.g, b.beta, m, L.state, b.y, s), "prefill gdn recurrence");
      ES_HIP(hipEventRecord(state_done_[slot][l], s), "prefill record");
      ES_HIP(launch_gdn_norm_gate_rows(b.y, b.z, L.gdn_norm, m, b.gated, s), "prefill gdn norm gate");
      ES_HIP(linear_rows(L.out, b.gated, m, routed, b.h, b.h, s), "prefill out_proj");
    } else {
      if (routed) {
        ES_HIP(linear_rows(L.q, b.u, m, routed, nullptr, b.qp, s), "prefill q");
        ES_HIP(linear_rows(L.k, b.u, m, routed, nullptr, b.kp, s), "prefill k");
        ES_HIP(linear_rows(L.v, b.u, m, routed, nullptr, b.vp, s), "prefill v");
      } else {
        const Q4 w[3] = {L.q, L.k, L.v};
        uint16_t* const y[3] = {b.qp, b.kp, b.vp};
        ES_HIP(launch_q4_gemm_stacked(w, y, 3, b.u, m, s), "prefill q|k|v");
      }
      AttnPrepRowsArgs a{b.qp, b.kp, b.vp, L.q_norm, L.k_norm, inv_freq_, pos0, m,
                         b.query, L.kcache, L.vcache, capacity_};
      ES_HIP(launch_attn_prep_rows(a, s), "prefill attention prepare");
      ES_HIP(launch_attn_prefill(b.query, L.kcache, L.vcache, pos0, m, capacity_, b.o, s), "prefill attention");
      // after the attention, which reads key blocks that may reach into the
      // next chunk's rows (masked, but read)
      ES_HIP(hipEventRecord(state_done_[slot][l], s), "prefill record");
      ES_HIP(launch_attn_gate_rows(b.o, b.qp, m, b.gated, s), "prefill attention gate");
      ES_HIP(linear_rows(L.o, b.gated, m, routed, b.h, b.h, s), "prefill o_proj");
    }
    ES_HIP(launch_rmsnorm_rows(b.h, L.post_norm, m, b.u, s), "prefill post norm");
    if (routed && m < qmv_row_limit(L.gate.n, L.gate.k)) {
      // gate and up as qmv_q4 rows, then swiglu_bf16 (model.rs:279-282); the
      // q|gate and raw-qkv buffers are free by now and hold the two outputs
      ES_HIP(launch_qmv_rows(L.gate, b.u, m, nullptr, b.raw, nullptr, s), "prefill gate");
      ES_HIP(launch_qmv_rows(L.up, b.u, m, nullptr, b.qp, nullptr, s), "prefill up");
      ES_HIP(launch_swiglu_rows(b.raw, b.qp, m * L.gate.n, b.act, s), "prefill swiglu");
    } else {
      ES_HIP(launch_q4_gemm_swiglu(L.gate, L.up, b.u, m, b.act, s), "prefill gate/up/swiglu");
    }
    ES_HIP(linear_rows(L.down, b.act, m, routed, b.h, b.h, s), "prefill down");
  }
  return 0;
}

// The prompt loop of Model::generate (model.rs:106-109): forwards of
// CHUNK = 2048 rows (model.rs:7) from position 0, so only the last one may be
// shorter. That last forward's row count r selects its routes: r == 1 runs the
// decode kernels (forward with rows == 1), and each linear with r below its
// row limit runs qmv_q4 rows (model.rs:189-198). Every other row takes the
// GEMM and the flash attention, whose per-row results do not depend on how
// rows are grouped into chunks, so those rows run in chunks of prefill_rows_.
// A cancellation check precedes each chunk (forward, model.rs:182).
int Engine::consume_prompt(const uint32_t* prompt, int n, std::string* err) {
  split_ = PromptSplit{};
  if (n <= 0) return 0;
  if (prefill_rows_ == 0) {
    split_.decode_rows = n;
    // each prompt step advances the step state to the next prompt token
    if (int rc = upload_state(0, 0, prompt[0], err)) return rc;
    return run_steps(kKindPrompt, 0, n, nullptr, nullptr, err);
  }
  int tail = n % kRefChunk;
  if (tail >= kMaxRowLimit) tail = 0;  // routes like a full forward
  const int body = n - tail;
  if (int rc = ensure_prefill_buffers(err)) return rc;
  const int chunk_rows = std::min(prefill_rows_, prefill_alloc_rows_);
  // the prefill streams start after the reset and the prompt upload on stream_
  ES_HIP(hipEventRecord(join_ev_[0], stream_), "prefill join");
  for (hipStream_t ps : pstream_) ES_HIP(hipStreamWaitEvent(ps, join_ev_[0], 0), "prefill join");
  auto join_back = [&]() -> int {
    for (int i = 0; i < kPrefillStreams; ++i) {
      ES_HIP(hipEventRecord(join_ev_[1 + i], pstream_[i]), "prefill join");
      ES_HIP(hipStreamWaitEvent(stream_, join_ev_[1 + i], 0), "prefill join");
    }
    return 0;
  };
  auto cancelled = [&]() -> bool {
    if (!cancelled_.load()) return false;
    for (hipStream_t ps : pstream_) (void)hipStreamSynchronize(ps);
    (void)hipStreamSynchronize(stream_);
    if (err) *err = "input disconnected";
    return true;
  };
  int pos = 0, chunk = 0;
  while (pos < body) {
    if (cancelled()) return 3;
    const int m = std::min(chunk_rows, body - pos);
    if (int rc = prefill_rows(pos, m, chunk % kPrefillStreams, chunk > 0, false, err)) {
      for (hipStream_t ps : pstream_) (void)hipStreamSynchronize(ps);
      return rc;
    }
    pos += m;
    ++chunk;
    ++split_.chunks;
  }
  if (tail > 0 && cancelled()) return 3;
  if (tail >= 2) {
    if (int rc = prefill_rows(pos, tail, chunk % kPrefillStreams, chunk > 0, true, err)) {
      for (hipStream_t ps : pstream_) (void)hipStreamSynchronize(ps);
      return rc;
    }
    pos += tail;
    split_.routed_rows = tail;
  }
  if (int rc = join_back()) return rc;
  if (tail == 1) {
    split_.decode_rows = 1;
    // the decode kernels on stream_, after the chunks
    if (int rc = upload_state(pos, 0, prompt[pos], err)) return rc;
    if (int rc = run_steps(kKindPrompt, pos, 1, nullptr, nullptr, err)) return rc;
  }
  ES_HIP(hipStreamSynchronize(stream_), "prefill sync");
  return 0;
}

int Engine::forced_decode(const uint32_t* tokens, int n, uint32_t* argmax_out,
                          uint16_t* logits_out, std::string* err) {
  if (n <= 0 || !tokens || !argmax_out) {
    if (err) *err = "invalid forced decode request";
    return 1;
  }
  if ((int64_t)position_ + n > capacity_) {
    if (err) *err = "context capacity exceeded";
    return 1;
  }
  for (int i = 0; i < n; ++i)
    if (tokens[i] >= (uint32_t)shape_.vocab) {
      if (err) *err = "token outside vocabulary";
      return 1;
    }
  ES_HIP(hipMemcpyAsync(forced_, tokens, (size_t)n * 4, hipMemcpyHostToDevice, stream_),
         "forced upload");
  if (int rc = upload_state(position_, 0, tokens[0], err)) return rc;
  if (int rc = run_steps(kKindDecode, position_, n, forced_, logits_out, err)) {
    reset_state();
    return rc;
  }
  ES_HIP(hipMemcpy(argmax_out, out_, (size_t)n * 4, hipMemcpyDeviceToHost), "argmax readback");
  position_ += n;
  pending_ = argmax_out[n - 1];
  has_pending_ = true;
  return 0;
}

int Engine::read_kv(int layer, int which, int pos0, int count, void* host, std::string* err) {
  if (layer < 0 || layer >= shape_.n_layers || !layers_[layer].attention || which < 0 ||
      which > 1 || pos0 < 0 || count < 0 || pos0 + count > capacity_ || !host) {
    if (err) *err = "invalid KV read";
    return 1;
  }
  const uint16_t* base = which == 0 ? layers_[layer].kcache : layers_[layer].vcache;
  // the copies run on the null stream: finish the engine stream's work first
  ES_HIP(hipStreamSynchronize(stream_), "sync");
  for (int h = 0; h < 2; ++h)
    ES_HIP(hipMemcpy(static_cast<uint16_t*>(host) + (size_t)h * count * 256,
                     base + ((size_t)h * capacity_ + pos0) * 256, (size_t)count * 256 * 2,
                     hipMemcpyDeviceToHost),
           "kv read");
  return 0;
}

int Engine::write_kv(int layer, int which, int pos0, int count, const void* host,
                     std::string* err) {
  if (layer < 0 || layer >= shape_.n_layers || !layers_[layer].attention || which < 0 ||
      which > 1 || pos0 < 0 || count < 0 || pos0 + count > capacity_ || !host) {
    if (err) *err = "invalid KV write";
    return 1;
  }
  uint16_t* base = which == 0 ? layers_[layer].kcache : layers_[layer].vcache;
  // the copies run on the null stream: finish the engine stream's work first
  ES_HIP(hipStreamSynchronize(stream_), "sync");
  for (int h = 0; h < 2; ++h)
    ES_HIP(hipMemcpy(base + ((size_t)h * capacity_ + pos0) * 256,
                     static_cast<const uint16_t*>(host) + (size_t)h * count * 256,
                     (size_t)count * 256 * 2, hipMemcpyHostToDevice),
           "kv write");
  return 0;
}

int Engine::read_gdn(int layer, void* ring_host, void* state_host, std::string* err) {
  if (layer < 0 || layer >= shape_.n_layers || layers_[layer].attention) {
    if (err) *err = "invalid GDN read";
    return 1;
  }
  ES_HIP(hipStreamSynchronize(stream_), "sync");
  if (ring_host)
    ES_HIP(hipMemcpy(ring_host, layers_[layer].ring, (size_t)4 * kConv * 2, hipMemcpyDeviceToHost),
           "ring read");
  if (state_host)
    ES_HIP(hipMemcpy(state_host, layers_[layer].state, (size_t)16 * 128 * 128 * 4,
                     hipMemcpyDeviceToHost),
           "state read");
  return 0;
}

int Engine::write_gdn(int layer, const void* ring_host, const void* state_host,
                      std::string* err) {
  if (layer < 0 || layer >= shape_.n_layers || layers_[layer].attention) {
    if (err) *err = "invalid GDN write";
    return 1;
  }
  ES_HIP(hipStreamSynchronize(stream_), "sync");
  if (ring_host)
    ES_HIP(hipMemcpy(layers_[layer].ring, ring_host, (size_t)4 * kConv * 2, hipMemcpyHostToDevice),
           "ring write");
  if (state_host)
    ES_HIP(hipMemcpy(layers_[layer].state, state_host, (size_t)16 * 128 * 128 * 4,
                     hipMemcpyHostToDevice),
           "state write");
  return 0;
}

int Engine::fill_synthetic(int length, uint64_t seed, uint32_t token, std::string* err) {
  if (length < 0 || length >= capacity_ || token >= (uint32_t)shape_.vocab) {
    if (err) *err = "invalid synthetic context";
    return 1;
  }
  uint64_t s = seed * 0x9E3779B97F4A7C15ull + 1;
  for (auto& L : layers_) {
    if (L.attention) {
      for (int h = 0; h < 2; ++h) {
        ES_HIP(launch_fill_normal_bf16(L.kcache + (size_t)h * capacity_ * 256,
                                       (size_t)length * 256, 1.0f, s++, stream_),
               "fill k");
        ES_HIP(launch_fill_normal_bf16(L.vcache + (size_t)h * capacity_ * 256,
                                       (size_t)length * 256, 1.0f, s++, stream_),
               "fill v");
      }
    } else {
      ES_HIP(launch_fill_normal_bf16(L.ring, (size_t)4 * kConv, 1.0f, s++, stream_), "fill ring");
      ES_HIP(launch_fill_normal_f32(L.state, (size_t)16 * 128 * 128, 0.1f, s++, stream_),
             "fill state");
    }
  }
  ES_HIP(hipStreamSynchronize(stream_), "fill sync");
  position_ = length;
  pending_ = token;
  has_pending_ = true;
  return 0;
}

int Engine::set_position(int position, uint32_t pending, std::string* err) {
  if (position < 0 || position >= capacity_ || pending >= (uint32_t)shape_.vocab) {
    if (err) *err = "invalid position";
    return 1;
  }
  position_ = position;
  pending_ = pending;
  has_pending_ = true;
  return 0;
}

int Engine::time_decode(int steps, int warmup, double* ms_total, std::string* err) {
  if (steps <= 0 || warmup < 0 || !has_pending_ ||
      (int64_t)position_ + steps + warmup > capacity_) {
    if (err) *err = "invalid timing request";
    return 1;
  }
  if (int rc = upload_state(position_, 0, pending_, err)) return rc;
  // capture every graph of the timed run before the clock starts
  for (const auto& [splits, n] : step_plan(position_ + warmup, steps))
    if (!graph(kKindDecode, splits, n, err)) return 2;
  if (int rc = launch_steps(kKindDecode, position_, warmup, err)) return rc;
  ES_HIP(hipStreamSynchronize(stream_), "warmup sync");
  hipEvent_t e0, e1;
  ES_HIP(hipEventCreate(&e0), "event");
  ES_HIP(hipEventCreate(&e1), "event");
  ES_HIP(hipEventRecord(e0, stream_), "record");
  if (int rc = launch_steps(kKindDecode, position_ + warmup, steps, err)) return rc;
  ES_HIP(hipEventRecord(e1, stream_), "record");
  ES_HIP(hipEventSynchronize(e1), "event sync");
  float ms = 0.0f;
  ES_HIP(hipEventElapsedTime(&ms, e0, e1), "elapsed");
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *ms_total = ms;
  uint32_t last = 0;
  ES_HIP(hipMemcpy(&last, out_ + (steps + warmup - 1), 4, hipMemcpyDeviceToHost), "readback");
  position_ += steps + warmup;
  pending_ = last;
  return check_device_error(err);
}

hipError_t Engine::launch_attention_part(const AttnArgs& a, int which) {
  hipError_t e = hipSuccess;
  if (which == 0 || which == 1) e = launch_attn_fused(a, stream_);
  if (e == hipSuccess && (which == 0 || which == 2)) e = launch_attn_merge(a, stream_);
  return e;
}

// layer < 0 rotates over every attention layer, so each launch streams a KV
// cache the previous launches did not touch (as in a decode step, where the
// six layers' caches together exceed the on-package cache); layer >= 0
// repeats one layer.
int Engine::time_attention(int layer, int reps, int which, double* ms_avg, std::string* err) {
  std::vector<int> att;
  for (int l = 0; l < shape_.n_layers; ++l)
    if (layers_[l].attention && (layer < 0 || l == layer)) att.push_back(l);
  if (att.empty() || layer >= shape_.n_layers || reps <= 0 || which < 0 || which > 2) {
    if (err) *err = "invalid attention timing request";
    return 1;
  }
  if (int rc = upload_state(position_, 0, pending_, err)) return rc;
  std::vector<AttnArgs> args;
  for (int l : att) args.push_back(attn_args(layers_[l], splits_for(position_ + 1)));
  // The timed launches write the K/V row of the current position, the row the
  // next decode step writes before anything reads it.
  for (const AttnArgs& a : args) ES_HIP(launch_attention_part(a, 0), "attn warmup");
  ES_HIP(hipStreamSynchronize(stream_), "sync");
  hipEvent_t e0, e1;
  ES_HIP(hipEventCreate(&e0), "event");
  ES_HIP(hipEventCreate(&e1), "event");
  ES_HIP(hipEventRecord(e0, stream_), "record");
  for (int i = 0; i < reps; ++i)
    ES_HIP(launch_attention_part(args[i % args.size()], which), "attn");
  ES_HIP(hipEventRecord(e1, stream_), "record");
  ES_HIP(hipEventSynchronize(e1), "sync");
  float ms = 0.0f;
  ES_HIP(hipEventElapsedTime(&ms, e0, e1), "elapsed");
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *ms_avg = ms / reps;
  return 0;
}

int Engine::time_head(int reps, double* ms_avg, std::string* err) {
  if (reps <= 0) {
    if (err) *err = "invalid head timing request";
    return 1;
  }
  HeadArgs h{};
  h.embed = embed_;
  h.h = h_;
  if (fused_mlp_) {  // the step's variant of the head
    h.h = hmid_;
    h.dpart = dpart_;
  }
  h.gain = final_norm_;
  h.logits = logits_;
  h.part = head_part_;
  uint32_t* tok = forced_;
  h.token_out = tok;
  ES_HIP(launch_head(h, stream_), "head warmup");
  ES_HIP(hipStreamSynchronize(stream_), "sync");
  hipEvent_t e0, e1;
  ES_HIP(hipEventCreate(&e0), "event");
  ES_HIP(hipEventCreate(&e1), "event");
  ES_HIP(hipEventRecord(e0, stream_), "record");
  for (int i = 0; i < reps; ++i) ES_HIP(launch_head(h, stream_), "head");
  ES_HIP(hipEventRecord(e1, stream_), "record");
  ES_HIP(hipEventSynchronize(e1), "sync");
  float ms = 0.0f;
  ES_HIP(hipEventElapsedTime(&ms, e0, e1), "elapsed");
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *ms_avg = ms / reps;
  return 0;
}

}  // namespace es
