// EngineSmith protocol v1 server (docs/protocol.md) over the engine C ABI,
// mirroring source/src/main.rs:10-53: a reader thread feeds a bounded queue
// and cancels the engine on stdin EOF; requests are answered in order, one
// JSON object per line, keys sorted as serde_json writes them.
//
// Usage: es_server --model DIR
// DIR is a checkpoint directory (config.json and *.safetensors, loaded and
// checked as Weights::load does, weights.rs:11-53), or, when it has no
// config.json, holds es_model.json {"seed": S, "n_layers": L, "vocab": V
// [, "capacity": C]} describing a seeded random-init model.
#include <atomic>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <fstream>
#include <iostream>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

#include "es_decode.h"
#include "es_json.hpp"

namespace {

using es::Json;
using es::parse_json;


void write_json(std::ostream& o, const Json& v) {
  switch (v.kind) {
    case Json::Null: o << "null"; break;
    case Json::Bool: o << (v.b ? "true" : "false"); break;
    case Json::Num: o << v.s; break;
    case Json::Str: {
      o << '"';
      for (unsigned char c : v.s) {
        if (c == '"') o << "\\\"";
        else if (c == '\\') o << "\\\\";
        else if (c == '\n') o << "\\n";
        else if (c == '\r') o << "\\r";
        else if (c == '\t') o << "\\t";
        else if (c < 0x20) { char b[8]; std::snprintf(b, sizeof b, "\\u%04x", c); o << b; }
        else o << c;
      }
      o << '"';
      break;
    }
    case Json::Arr: {
      o << '[';
      for (size_t i = 0; i < v.arr.size(); ++i) {
        if (i) o << ',';
        write_json(o, v.arr[i]);
      }
      o << ']';
      break;
    }
    case Json::Obj: {
      o << '{';
      bool first = true;
      for (const auto& kv : v.obj) {
        if (!first) o << ',';
        first = false;
        Json k;
        k.kind = Json::Str;
        k.s = kv.first;
        write_json(o, k);
        o << ':';
        write_json(o, kv.second);
      }
      o << '}';
      break;
    }
  }
}

Json jstr(const std::string& s) { Json j; j.kind = Json::Str; j.s = s; return j; }
Json jbool(bool b) { Json j; j.kind = Json::Bool; j.b = b; return j; }
Json jint(long long x) { Json j; j.kind = Json::Num; j.is_int = true; j.i = x; j.s = std::to_string(x); return j; }

// ---- bounded line channel (main.rs:17-25) ----
struct Channel {
  std::mutex m;
  std::condition_variable cv;
  std::deque<std::string> q;
  bool closed = false;
  void push(std::string s) {
    std::unique_lock<std::mutex> l(m);
    cv.wait(l, [&] { return q.size() < 1 || closed; });
    q.push_back(std::move(s));
    cv.notify_all();
  }
  bool pop(std::string& s) {
    std::unique_lock<std::mutex> l(m);
    cv.wait(l, [&] { return !q.empty() || closed; });
    if (q.empty()) return false;
    s = std::move(q.front());
    q.pop_front();
    cv.notify_all();
    return true;
  }
  void close() {
    std::lock_guard<std::mutex> l(m);
    closed = true;
    cv.notify_all();
  }
};

bool read_file(const std::string& path, std::string& out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  std::stringstream ss;
  ss << f.rdbuf();
  out = ss.str();
  return true;
}

int die(const std::string& msg) {
  std::fprintf(stderr, "engine: %s\n", msg.c_str());
  return 1;
}

}  // namespace

int main(int argc, char** argv) {
  std::string model_dir;
  for (int i = 1; i < argc; ++i) {
    std::string a = argv[i];
    if (a == "--model" && i + 1 < argc) model_dir = argv[++i];
    else return die("unknown argument " + a);
  }
  if (model_dir.empty()) return die("--model MODEL_DIR required");
  std::string text, err;
  int n_layers = 24, vocab = 248320, capacity = 262144;  // model.rs:8-9
  std::vector<uint8_t> blob;
  size_t bytes = 0;
  if (read_file(model_dir + "/config.json", text) || !read_file(model_dir + "/es_model.json", text)) {
    // checkpoint directory (Model::load, model.rs:38-79)
    if (es_checkpoint_config(model_dir.c_str(), &n_layers, &vocab) != ES_OK) return die(es_last_error());
    bytes = es_weights_total_bytes(n_layers, vocab);
    blob.resize(bytes);
    if (es_checkpoint_load(model_dir.c_str(), n_layers, vocab, blob.data(), bytes) != ES_OK)
      return die(es_last_error());
  } else {
    Json cfg;
    if (!parse_json(text, cfg, err) || cfg.kind != Json::Obj) return die("invalid es_model.json: " + err);
    auto num = [&](const char* k, long long def) -> long long {
      const Json* v = cfg.get(k);
      return v && v->kind == Json::Num ? v->i : def;
    };
    n_layers = (int)num("n_layers", 24);
    vocab = (int)num("vocab", 248320);
    capacity = (int)num("capacity", 262144);
    const unsigned long long seed = (unsigned long long)num("seed", 0);
    bytes = es_weights_total_bytes(n_layers, vocab);
    if (!bytes) return die("unsupported model configuration");
    blob.resize(bytes);
    if (es_weights_random(n_layers, vocab, seed, blob.data(), bytes, 0) != ES_OK)
      return die(es_last_error());
  }
  es_engine* engine = es_engine_create(blob.data(), bytes, n_layers, vocab, capacity);
  if (!engine) return die(es_last_error());
  std::vector<uint8_t>().swap(blob);

  Channel ch;
  std::atomic<bool> disconnected{false};
  std::thread reader([&] {
    std::string line;
    while (std::getline(std::cin, line)) ch.push(line);
    // Disconnect stops inference after the currently submitted GPU work.
    disconnected.store(true);
    es_engine_cancel(engine);
    ch.close();
  });
  reader.detach();

  std::string line;
  int exit_code = 0;
  std::vector<uint32_t> out;
  while (ch.pop(line)) {
    if (disconnected.load()) break;
    Json req;
    if (!parse_json(line, req, err)) {
      exit_code = die("invalid request JSON: " + err);
      break;
    }
    Json reply;
    reply.kind = Json::Obj;
    const Json* id = req.get("id");
    reply.obj["id"] = id ? *id : Json();
    std::string error;
    const Json* op = req.get("op");
    if (!op || op->kind != Json::Str) {
      error = "missing op";
    } else if (op->s == "hello") {
      reply.obj["protocol"] = jint(1);
    } else if (op->s == "generate") {
      const Json* prompt = req.get("prompt");
      const Json* mt = req.get("max_tokens");
      const Json* rs = req.get("reset");
      std::vector<uint32_t> ids;
      if (!prompt || prompt->kind != Json::Arr) error = "missing prompt";
      else {
        ids.reserve(prompt->arr.size());
        for (const Json& x : prompt->arr) {
          if (x.kind != Json::Num || !x.is_int || x.neg || x.i > 0xffffffffLL) {
            error = "invalid token";
            break;
          }
          ids.push_back((uint32_t)x.i);
        }
      }
      if (error.empty() && (!mt || mt->kind != Json::Num || !mt->is_int || mt->neg))
        error = "missing max_tokens";
      if (error.empty() && (!rs || rs->kind != Json::Bool)) error = "missing reset";
      if (error.empty()) {
        long long count = mt->i;
        if (count > 0x7fffffffLL) count = 0x7fffffffLL;
        out.assign(count > 0 && count <= (1 << 22) ? (size_t)count : 1, 0);
        int rc = es_engine_generate(engine, ids.data(), (int)ids.size(), (int)count, rs->b ? 1 : 0,
                                    out.data());
        if (rc == ES_ERR_CANCELLED) break;
        if (rc != ES_OK) error = es_last_error();
        else {
          Json toks;
          toks.kind = Json::Arr;
          toks.arr.reserve(count);
          for (long long i = 0; i < count; ++i) toks.arr.push_back(jint(out[i]));
          reply.obj["tokens"] = std::move(toks);
        }
      }
    } else {
      error = "unknown operation " + op->s;
    }
    if (disconnected.load()) break;
    if (!error.empty()) {
      reply.obj.erase("protocol");
      reply.obj.erase("tokens");
      reply.obj["ok"] = jbool(false);
      reply.obj["error"] = jstr(error);
    } else {
      reply.obj["ok"] = jbool(true);
    }
    std::ostringstream os;
    write_json(os, reply);
    os << '\n';
    const std::string s = os.str();
    std::fwrite(s.data(), 1, s.size(), stdout);
    std::fflush(stdout);
  }
  es_engine_destroy(engine);
  std::fflush(stdout);
  std::_Exit(exit_code);
}
