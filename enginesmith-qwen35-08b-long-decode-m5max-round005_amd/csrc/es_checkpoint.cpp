// Checkpoint loading: config.json validation and the safetensors files of a
// model directory into the weight blob (weights.rs:11-53, model.rs:38-79).
// The same checks as the reference, in the same order and with its messages:
// every *.safetensors file of the directory (sorted by path) is read, tensors
// outside language_model.model.* are skipped, dtypes are U32 / F32 / BF16,
// each tensor's byte range must lie inside the file's data section and match
// its shape, no name may repeat, the text tensor count must be the model's
// (694 for 24 layers), and every tensor the model takes must exist with the
// expected shape and dtype. Files are memory-mapped, not read whole.
#include "es_checkpoint.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <dirent.h>
#include <map>
#include <memory>

#include "es_json.hpp"
#include "es_weights.hpp"

namespace es {
namespace {

const char* kPrefix = "language_model.model.";

struct Mapped {
  void* base = nullptr;
  size_t size = 0;
  int fd = -1;
  ~Mapped() {
    if (base && base != MAP_FAILED) munmap(base, size);
    if (fd >= 0) close(fd);
  }
};

struct Entry {
  const uint8_t* data;
  uint64_t bytes;
  std::string dtype;
  std::vector<int64_t> shape;
};

bool read_text(const std::string& path, std::string& out, std::string* err) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) {
    if (err) *err = path + ": " + std::strerror(errno);
    return false;
  }
  char buf[65536];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) out.append(buf, n);
  std::fclose(f);
  return true;
}

bool json_u64(const Json* v, uint64_t* out) {
  if (!v || v->kind != Json::Num || !v->is_int || v->neg) return false;
  *out = (uint64_t)v->i;
  return true;
}

const char* dtype_name(DType d) { return d == kU32 ? "U32" : d == kBF16 ? "BF16" : "F32"; }

bool fail(std::string* err, const std::string& m) {
  if (err) *err = m;
  return false;
}

}  // namespace

bool checkpoint_config(const std::string& dir, int* n_layers, int* vocab, std::string* err) {
  std::string text;
  if (!read_text(dir + "/config.json", text, err)) return false;
  Json cfg;
  std::string perr;
  if (!parse_json(text, cfg, perr)) return fail(err, "config.json: " + perr);
  const Json* tc = cfg.kind == Json::Obj ? cfg.get("text_config") : nullptr;
  auto is = [&](const char* k, long long want) {
    const Json* v = tc && tc->kind == Json::Obj ? tc->get(k) : nullptr;
    return v && v->kind == Json::Num && v->is_int && v->i == want;
  };
  if (!(is("hidden_size", 1024) && is("num_hidden_layers", 24) && is("vocab_size", 248320)))
    return fail(err, "unsupported model configuration");
  *n_layers = 24;
  *vocab = 248320;
  return true;
}

bool checkpoint_load(const std::string& dir, int n_layers, int vocab, void* blob, uint64_t bytes,
                     std::string* err) {
  uint64_t total = 0;
  const std::vector<TensorDesc> layout = weight_layout(ModelShape{n_layers, vocab}, &total);
  if (!blob || bytes < total) return fail(err, "weight blob too small");

  std::vector<std::string> files;
  DIR* d = opendir(dir.c_str());
  if (!d) return fail(err, dir + ": " + std::strerror(errno));
  while (dirent* e = readdir(d)) {
    const std::string n = e->d_name;
    const std::string ext = ".safetensors";
    if (n.size() > ext.size() && n.compare(n.size() - ext.size(), ext.size(), ext) == 0)
      files.push_back(dir + "/" + n);
  }
  closedir(d);
  std::sort(files.begin(), files.end());
  if (files.empty()) return fail(err, "no safetensors weights");

  std::vector<std::unique_ptr<Mapped>> maps;
  std::map<std::string, Entry> tensors;
  for (const std::string& path : files) {
    auto m = std::make_unique<Mapped>();
    m->fd = open(path.c_str(), O_RDONLY);
    struct stat st {};
    if (m->fd < 0 || fstat(m->fd, &st) != 0) return fail(err, "read " + path + ": " + std::strerror(errno));
    m->size = (size_t)st.st_size;
    if (m->size < 8) return fail(err, "short safetensors file");
    m->base = mmap(nullptr, m->size, PROT_READ, MAP_PRIVATE, m->fd, 0);
    if (m->base == MAP_FAILED) return fail(err, "read " + path + ": " + std::strerror(errno));
    const uint8_t* bytes8 = static_cast<const uint8_t*>(m->base);
    uint64_t n = 0;
    std::memcpy(&n, bytes8, 8);  // little-endian host
    if (n > m->size - 8) return fail(err, "invalid safetensors header");
    Json header;
    std::string perr;
    if (!parse_json(std::string(reinterpret_cast<const char*>(bytes8 + 8), (size_t)n), header, perr))
      return fail(err, "invalid header: " + perr);
    if (header.kind != Json::Obj) return fail(err, "invalid header");
    const uint64_t data_len = m->size - 8 - n;
    const uint8_t* data = bytes8 + 8 + n;
    for (const auto& kv : header.obj) {
      const std::string& full = kv.first;
      if (full == "__metadata__") continue;
      if (full.compare(0, std::strlen(kPrefix), kPrefix) != 0) continue;
      const std::string name = full.substr(std::strlen(kPrefix));
      const Json& v = kv.second;
      const Json* dt = v.kind == Json::Obj ? v.get("dtype") : nullptr;
      if (!dt || dt->kind != Json::Str) return fail(err, "missing dtype");
      uint64_t elem = 0;
      if (dt->s == "U32" || dt->s == "F32") elem = 4;
      else if (dt->s == "BF16") elem = 2;
      else return fail(err, "unsupported dtype " + dt->s);
      const Json* sh = v.get("shape");
      if (!sh || sh->kind != Json::Arr) return fail(err, "missing shape");
      std::vector<int64_t> shape;
      uint64_t count = 1;
      for (const Json& x : sh->arr) {
        uint64_t u;
        if (!json_u64(&x, &u)) return fail(err, "invalid shape");
        shape.push_back((int64_t)u);
        count *= u;
      }
      const Json* off = v.get("data_offsets");
      uint64_t start = 0, end = 0;
      if (!off || off->kind != Json::Arr || off->arr.size() < 1 || !json_u64(&off->arr[0], &start))
        return fail(err, "invalid offset");
      if (off->arr.size() < 2 || !json_u64(&off->arr[1], &end)) return fail(err, "invalid offset");
      if (!(end >= start && end <= data_len && end - start == count * elem))
        return fail(err, "tensor bounds: " + name);
      if (!tensors.emplace(name, Entry{data + start, end - start, dt->s, shape}).second)
        return fail(err, "duplicate tensor " + name);
    }
    maps.push_back(std::move(m));
  }
  if (tensors.size() != layout.size())
    return fail(err, "expected " + std::to_string(layout.size()) + " text tensors, got " +
                         std::to_string(tensors.size()));

  // The model takes its tensors in the reference's order (embedding, final
  // norm, then per layer), so the first missing or mismatched one is the one
  // the reference reports.
  std::memset(blob, 0, total);  // alignment gaps between tensors read as zero
  for (const TensorDesc& t : layout) {
    auto it = tensors.find(t.name);
    if (it == tensors.end()) return fail(err, "missing " + t.name);
    if (it->second.shape != t.shape || it->second.dtype != dtype_name(t.dtype) || it->second.bytes != t.bytes)
      return fail(err, "wrong shape/dtype for " + t.name);
    std::memcpy(static_cast<uint8_t*>(blob) + t.offset, it->second.data, t.bytes);
    tensors.erase(it);
  }
  if (!tensors.empty()) {
    std::string names;
    for (const auto& kv : tensors) names += (names.empty() ? "" : ", ") + kv.first;
    return fail(err, "unused text weights: " + names);
  }
  return true;
}

}  // namespace es
