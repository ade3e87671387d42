// kernel_cache.cpp -- (gpu, op, shape) -> validated tuning entry + the code
// object that implements it, persisted as two JSON files.
//
// Behaviour follows lib/Runtime/KernelCache.cpp of the reference: a miss and
// an unvalidated entry are the only non-served outcomes, each with an
// actionable message (:84-107); binaries are keyed like the entries and must
// back one (:296-306); Persist/LoadPersisted write and read
// <dir>/tuning_db.json and <dir>/binaries.json (:321-369), loading into
// temporaries so a failure leaves the cache untouched; InvalidateStale drops
// every entry whose binary is missing or re-hashes differently (:371-392).
#include <filesystem>
#include <fstream>
#include <set>
#include <sstream>

#include "../../../include/polykernel_amd_runtime.hpp"
#include "json.hpp"

namespace pk::runtime {

namespace {

constexpr int kBinariesVersion = 1;
constexpr const char *kTuningFile = "/tuning_db.json";
constexpr const char *kBinariesFile = "/binaries.json";

bool ReadFile(const std::string &path, std::string &out, std::string &error, const char *what = "") {
  std::ifstream in(path, std::ios::binary);
  if (!in) {
    error = std::string("cannot read ") + what + path;
    return false;
  }
  std::ostringstream ss;
  ss << in.rdbuf();
  if (in.bad()) {
    error = std::string("cannot read ") + what + path;
    return false;
  }
  out = ss.str();
  return true;
}

bool WriteFile(const std::string &path, const std::string &content, std::string &error) {
  // write-then-rename so a reader never sees a half-written file
  const std::string tmp = path + ".tmp";
  {
    std::ofstream out(tmp, std::ios::binary | std::ios::trunc);
    if (!out) {
      error = "cannot open " + tmp + " for writing";
      return false;
    }
    out << content;
    out.flush();
    if (!out) {
      error = "write failed for " + tmp;
      return false;
    }
  }
  std::error_code ec;
  std::filesystem::rename(tmp, path, ec);
  if (ec) {
    error = "cannot rename " + tmp + " to " + path + ": " + ec.message();
    return false;
  }
  return true;
}

const json::Value *Req(const json::Object &o, const char *key, const std::string &path, const char *what,
                       std::string &error) {
  const json::Value *v = json::Get(o, key);
  if (v == nullptr) error = path + "." + key + ": missing required " + what + " field";
  return v;
}

bool ReqString(const json::Object &o, const char *key, const std::string &path, std::string &out,
               std::string &error) {
  const json::Value *v = Req(o, key, path, "string", error);
  if (v == nullptr) return false;
  if (v->as_string() == nullptr) {
    error = path + "." + key + ": expected a string";
    return false;
  }
  out = *v->as_string();
  return true;
}

bool ReqInt(const json::Object &o, const char *key, const std::string &path, int64_t &out, std::string &error) {
  const json::Value *v = Req(o, key, path, "integer", error);
  if (v == nullptr) return false;
  const auto i = v->as_integer();
  if (!i) {
    error = path + "." + key + ": expected an integer";
    return false;
  }
  out = *i;
  return true;
}

std::string SerializeBinaries(const autotune::AmdTuningDb &db, const std::map<std::string, CachedBinary> &bins) {
  json::Array arr;
  for (const std::string &ns : db.Namespaces()) {
    for (const CacheEntry &e : db.Entries(ns)) {
      const auto it = bins.find(FormatKey(e.gpu, e.op, e.shape));
      if (it == bins.end()) continue;
      json::Object shape{{"M", json::Value((long long)e.shape.m)},
                         {"N", json::Value((long long)e.shape.n)},
                         {"K", json::Value((long long)e.shape.k)},
                         {"dtype", e.shape.dtype}};
      arr.push_back(json::Object{{"gpu", e.gpu},
                                 {"op", e.op},
                                 {"shape", json::Value(std::move(shape))},
                                 {"so_path", it->second.so_path},
                                 {"kernel_hash", it->second.kernel_hash}});
    }
  }
  return json::Serialize(json::Object{{"version", kBinariesVersion}, {"binaries", json::Value(std::move(arr))}});
}

// Error paths are unprefixed; the caller adds "binaries.json: ".
bool ParseBinaries(std::string_view text, const autotune::AmdTuningDb &db,
                   std::map<std::string, CachedBinary> &out, std::string &error) {
  json::ParseResult p = json::Parse(text);
  if (!p.ok()) {
    error = "malformed JSON: " + p.error;
    return false;
  }
  const json::Object *root = p.value->as_object();
  if (root == nullptr) {
    error = "root: expected a JSON object (the binaries envelope)";
    return false;
  }
  int64_t version = 0;
  if (!ReqInt(*root, "version", "root", version, error)) return false;
  if (version != kBinariesVersion) {
    error = "root.version: unsupported binaries version " + std::to_string(version) + " (expected " +
            std::to_string(kBinariesVersion) + ")";
    return false;
  }
  const json::Value *bv = Req(*root, "binaries", "root", "array", error);
  if (bv == nullptr) return false;
  const json::Array *arr = bv->as_array();
  if (arr == nullptr) {
    error = "root.binaries: expected an array";
    return false;
  }
  for (size_t i = 0; i < arr->size(); ++i) {
    const std::string path = "binaries[" + std::to_string(i) + "]";
    const json::Object *o = (*arr)[i].as_object();
    if (o == nullptr) {
      error = path + ": expected an object";
      return false;
    }
    std::string gpu, op, so_path, hash;
    Shape shape;
    if (!ReqString(*o, "gpu", path, gpu, error) || !ReqString(*o, "op", path, op, error)) return false;
    const json::Value *sv = Req(*o, "shape", path, "object", error);
    if (sv == nullptr) return false;
    const json::Object *so = sv->as_object();
    if (so == nullptr) {
      error = path + ".shape: expected an object";
      return false;
    }
    const std::string sp = path + ".shape";
    if (!ReqInt(*so, "M", sp, shape.m, error) || !ReqInt(*so, "N", sp, shape.n, error) ||
        !ReqInt(*so, "K", sp, shape.k, error) || !ReqString(*so, "dtype", sp, shape.dtype, error))
      return false;
    if (!ReqString(*o, "so_path", path, so_path, error) || !ReqString(*o, "kernel_hash", path, hash, error))
      return false;
    if (!db.Get(gpu, op, shape)) {
      error = path + ": no tuning entry for " + FormatKey(gpu, op, shape) +
              " (a binary must back a present tuning entry)";
      return false;
    }
    out[FormatKey(gpu, op, shape)] = CachedBinary{std::move(so_path), std::move(hash)};
  }
  return true;
}

}  // namespace

std::string FormatKey(std::string_view gpu, std::string_view op, const Shape &s) {
  return std::string(gpu) + "/" + std::string(op) + "/M=" + std::to_string(s.m) + ",N=" + std::to_string(s.n) +
         ",K=" + std::to_string(s.k) + "," + s.dtype;
}

bool HashFile(std::string_view path, std::string &hash_out, std::string &error) {
  std::ifstream in(std::string(path), std::ios::binary);
  if (!in) {
    error = "cannot read binary " + std::string(path);
    return false;
  }
  // The reference's seed (lib/Runtime/KernelCache.cpp:56): one decimal digit
  // short of the published FNV-1a 64 offset basis 14695981039346656037, kept
  // so that hashes agree with the binaries.json files the reference writes.
  uint64_t h = 1469598103934665603ull;
  char buf[1 << 16];
  while (in) {
    in.read(buf, sizeof buf);
    const std::streamsize n = in.gcount();
    for (std::streamsize i = 0; i < n; ++i) {
      h ^= static_cast<unsigned char>(buf[i]);
      h *= 1099511628211ull;  // FNV-1a 64 prime
    }
  }
  if (in.bad()) {
    error = "cannot read binary " + std::string(path);
    return false;
  }
  static const char kHex[] = "0123456789abcdef";
  std::string hex(16, '0');
  for (int i = 15; i >= 0; --i, h >>= 4) hex[i] = kHex[h & 15];
  hash_out = std::move(hex);
  return true;
}

bool KernelCache::LoadTuningCache(std::string_view text, std::string &error) {
  autotune::AmdTuningDbParseResult p = autotune::AmdTuningDb::Parse(text);
  if (!p.ok()) {
    error = std::move(p.error);
    return false;
  }
  db_ = std::move(*p.db);
  // binaries must keep backing an entry
  for (auto it = binaries_.begin(); it != binaries_.end();) {
    bool backed = false;
    for (const std::string &ns : db_.Namespaces()) {
      for (const CacheEntry &e : db_.Entries(ns))
        if (FormatKey(e.gpu, e.op, e.shape) == it->first) backed = true;
    }
    it = backed ? std::next(it) : binaries_.erase(it);
  }
  return true;
}

bool KernelCache::Put(CacheEntry entry) { return db_.Put(std::move(entry)); }

SelectionResult KernelCache::Select(std::string_view gpu, std::string_view op, const Shape &shape) const {
  SelectionResult r;
  std::optional<CacheEntry> e = db_.Get(gpu, op, shape);
  if (!e) {
    r.error = "no tuned kernel for " + FormatKey(gpu, op, shape) +
              "; run the autotuner (polykernel_amd.autotune) to populate the cache";
    return r;
  }
  if (!e->validated) {
    r.error = "cached entry for " + FormatKey(gpu, op, shape) +
              " is not validated; run the autotuner to produce a correctness-gated variant";
    return r;
  }
  r.entry = std::move(e);
  return r;
}

bool KernelCache::PutBinary(std::string_view gpu, std::string_view op, const Shape &shape, CachedBinary binary) {
  if (gpu.empty() || !db_.Get(gpu, op, shape)) return false;
  binaries_[FormatKey(gpu, op, shape)] = std::move(binary);
  return true;
}

std::optional<CachedBinary> KernelCache::GetBinary(std::string_view gpu, std::string_view op,
                                                   const Shape &shape) const {
  const auto it = binaries_.find(FormatKey(gpu, op, shape));
  if (it == binaries_.end()) return std::nullopt;
  return it->second;
}

bool KernelCache::Persist(std::string_view cache_dir, std::string &error) const {
  const std::string dir(cache_dir);
  std::error_code ec;
  std::filesystem::create_directories(dir, ec);
  if (ec) {
    error = "cannot create cache dir " + dir + ": " + ec.message();
    return false;
  }
  return WriteFile(dir + kTuningFile, db_.Serialize(), error) &&
         WriteFile(dir + kBinariesFile, SerializeBinaries(db_, binaries_), error);
}

bool KernelCache::LoadPersisted(std::string_view cache_dir, std::string &error) {
  const std::string dir(cache_dir);
  std::string tuning, bins_text;
  if (!ReadFile(dir + kTuningFile, tuning, error) || !ReadFile(dir + kBinariesFile, bins_text, error))
    return false;
  autotune::AmdTuningDbParseResult p = autotune::AmdTuningDb::Parse(tuning);
  if (!p.ok()) {
    error = "tuning_db.json: " + p.error;
    return false;
  }
  std::map<std::string, CachedBinary> bins;
  if (!ParseBinaries(bins_text, *p.db, bins, error)) {
    error = "binaries.json: " + error;
    return false;
  }
  db_ = std::move(*p.db);
  binaries_ = std::move(bins);
  return true;
}

std::size_t KernelCache::InvalidateStale() {
  std::set<std::string> stale;
  for (const auto &[key, bin] : binaries_) {
    std::string hash, err;
    if (!HashFile(bin.so_path, hash, err) || hash != bin.kernel_hash) stale.insert(key);
  }
  if (stale.empty()) return 0;
  autotune::AmdTuningDb fresh;
  for (const std::string &ns : db_.Namespaces())
    for (const CacheEntry &e : db_.Entries(ns))
      if (!stale.count(FormatKey(e.gpu, e.op, e.shape))) fresh.Put(e);
  db_ = std::move(fresh);
  for (const std::string &k : stale) binaries_.erase(k);
  return stale.size();
}

std::vector<std::pair<std::string, SelectionResult>> KernelCache::SelectPerGpu(const std::vector<std::string> &gpus,
                                                                               std::string_view op,
                                                                               const Shape &shape) const {
  std::vector<std::pair<std::string, SelectionResult>> out;
  out.reserve(gpus.size());
  for (const std::string &g : gpus) out.emplace_back(g, Select(g, op, shape));
  return out;
}

}  // namespace pk::runtime
