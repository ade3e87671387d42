// tuning.cpp -- the tuning-cache document (tuning/schema.json), the
// gpu-partitioned tuning DB, and the correctness gate.
//
// Parsing is strict in the reference's way (lib/Autotune/TuningCache.cpp:
// 27-305): every required field must be present with its JSON type, errors
// name the field path ("entries[2].best.block_k: expected an integer"), the
// envelope version must be 1 and time_ms is the one nullable field.  Members
// the schema does not name are ignored, as the reference parser ignores them.
#include <algorithm>
#include <cmath>

#include "internal.hpp"

namespace pk::autotune {

namespace {

using json::Object;
using json::Value;

bool Field(const Object &obj, const char *key, const std::string &path, const char *what,
           const Value *&v, std::string &error) {
  v = json::Get(obj, key);
  if (v == nullptr) {
    error = path + "." + key + ": missing required " + what + " field";
    return false;
  }
  return true;
}

bool GetString(const Object &obj, const char *key, const std::string &path, std::string &out,
               std::string &error) {
  const Value *v;
  if (!Field(obj, key, path, "string", v, error)) return false;
  const std::string *s = v->as_string();
  if (s == nullptr) {
    error = path + "." + key + ": expected a string";
    return false;
  }
  out = *s;
  return true;
}

bool GetInt(const Object &obj, const char *key, const std::string &path, int64_t &out, std::string &error) {
  const Value *v;
  if (!Field(obj, key, path, "integer", v, error)) return false;
  const auto i = v->as_integer();
  if (!i) {
    error = path + "." + key + ": expected an integer";
    return false;
  }
  out = *i;
  return true;
}

bool GetInt32(const Object &obj, const char *key, const std::string &path, int &out, std::string &error) {
  int64_t v = 0;
  if (!GetInt(obj, key, path, v, error)) return false;
  if (v < INT32_MIN || v > INT32_MAX) {
    error = path + "." + key + ": integer out of range";
    return false;
  }
  out = static_cast<int>(v);
  return true;
}

bool GetDouble(const Object &obj, const char *key, const std::string &path, double &out, std::string &error) {
  const Value *v;
  if (!Field(obj, key, path, "number", v, error)) return false;
  const auto d = v->as_number();
  if (!d) {
    error = path + "." + key + ": expected a number";
    return false;
  }
  out = *d;
  return true;
}

bool GetBool(const Object &obj, const char *key, const std::string &path, bool &out, std::string &error) {
  const Value *v;
  if (!Field(obj, key, path, "boolean", v, error)) return false;
  const auto b = v->as_bool();
  if (!b) {
    error = path + "." + key + ": expected a boolean";
    return false;
  }
  out = *b;
  return true;
}

bool GetObject(const Object &obj, const char *key, const std::string &path, const Object *&out,
               std::string &error) {
  const Value *v;
  if (!Field(obj, key, path, "object", v, error)) return false;
  out = v->as_object();
  if (out == nullptr) {
    error = path + "." + key + ": expected an object";
    return false;
  }
  return true;
}

bool ParseShape(const Object &o, const std::string &path, Shape &s, std::string &error) {
  return GetInt(o, "M", path, s.m, error) && GetInt(o, "N", path, s.n, error) &&
         GetInt(o, "K", path, s.k, error) && GetString(o, "dtype", path, s.dtype, error);
}

bool ParseConfig(const Object &o, const std::string &path, Config &c, std::string &error) {
  return GetInt32(o, "block_m", path, c.block_m, error) && GetInt32(o, "block_n", path, c.block_n, error) &&
         GetInt32(o, "block_k", path, c.block_k, error) && GetInt32(o, "num_warps", path, c.num_warps, error) &&
         GetInt32(o, "vector_width", path, c.vector_width, error) &&
         GetInt32(o, "unroll", path, c.unroll, error) &&
         GetInt32(o, "shared_memory_stages", path, c.shared_memory_stages, error);
}

bool ParseEntry(const Object &o, const std::string &path, CacheEntry &e, std::string &error) {
  if (!GetString(o, "gpu", path, e.gpu, error) || !GetString(o, "op", path, e.op, error)) return false;
  const Object *shape = nullptr, *best = nullptr, *corr = nullptr;
  if (!GetObject(o, "shape", path, shape, error) || !ParseShape(*shape, path + ".shape", e.shape, error))
    return false;
  if (!GetObject(o, "best", path, best, error) || !ParseConfig(*best, path + ".best", e.best, error))
    return false;
  if (!GetString(o, "scored_by", path, e.scored_by, error)) return false;
  const Value *t = json::Get(o, "time_ms");
  if (t == nullptr) {
    error = path + ".time_ms: missing required field (use null for a compile-time-model score)";
    return false;
  }
  if (t->is_null()) {
    e.time_ms.reset();
  } else if (const auto d = t->as_number()) {
    e.time_ms = *d;
  } else {
    error = path + ".time_ms: expected a number or null";
    return false;
  }
  if (!GetBool(o, "validated", path, e.validated, error)) return false;
  if (!GetObject(o, "correctness", path, corr, error)) return false;
  const std::string cp = path + ".correctness";
  return GetDouble(*corr, "cosine", cp, e.correctness.cosine, error) &&
         GetDouble(*corr, "max_rel_err", cp, e.correctness.max_rel_err, error) &&
         GetDouble(*corr, "pcc", cp, e.correctness.pcc, error);
}


}  // namespace

namespace detail {

Value ShapeJson(const Shape &s) {
  return Object{{"M", Value((long long)s.m)}, {"N", Value((long long)s.n)}, {"K", Value((long long)s.k)},
                {"dtype", Value(s.dtype)}};
}

Value ConfigJson(const Config &c) {
  return Object{{"block_m", c.block_m},     {"block_n", c.block_n},           {"block_k", c.block_k},
                {"num_warps", c.num_warps}, {"vector_width", c.vector_width}, {"unroll", c.unroll},
                {"shared_memory_stages", c.shared_memory_stages}};
}

Value CorrectnessJson(const Correctness &c) {
  return Object{{"cosine", c.cosine}, {"max_rel_err", c.max_rel_err}, {"pcc", c.pcc}};
}

Value EntryJson(const CacheEntry &e) {
  return Object{{"gpu", e.gpu},
                {"op", e.op},
                {"shape", ShapeJson(e.shape)},
                {"best", ConfigJson(e.best)},
                {"scored_by", e.scored_by},
                {"time_ms", e.time_ms ? Value(*e.time_ms) : Value()},
                {"validated", e.validated},
                {"correctness", CorrectnessJson(e.correctness)}};
}

}  // namespace detail

std::string ToString(const Config &c) {
  return "block_m=" + std::to_string(c.block_m) + " block_n=" + std::to_string(c.block_n) +
         " block_k=" + std::to_string(c.block_k) + " num_warps=" + std::to_string(c.num_warps) +
         " vector_width=" + std::to_string(c.vector_width) + " unroll=" + std::to_string(c.unroll) +
         " shared_memory_stages=" + std::to_string(c.shared_memory_stages);
}

TuningCacheParseResult ParseTuningCache(std::string_view text) {
  TuningCacheParseResult r;
  json::ParseResult p = json::Parse(text);
  if (!p.ok()) {
    r.error = "malformed JSON: " + p.error;
    return r;
  }
  const Object *root = p.value->as_object();
  if (root == nullptr) {
    r.error = "root: expected a JSON object (the versioned envelope)";
    return r;
  }
  TuningCache cache;
  int64_t version = 0;
  if (!GetInt(*root, "version", "root", version, r.error)) return r;
  if (version != kTuningCacheVersion) {
    r.error = "root.version: unsupported schema version " + std::to_string(version) + " (expected " +
              std::to_string(kTuningCacheVersion) + ")";
    return r;
  }
  const Value *ev = json::Get(*root, "entries");
  if (ev == nullptr) {
    r.error = "root.entries: missing required array field";
    return r;
  }
  const json::Array *arr = ev->as_array();
  if (arr == nullptr) {
    r.error = "root.entries: expected an array";
    return r;
  }
  cache.entries.reserve(arr->size());
  for (size_t i = 0; i < arr->size(); ++i) {
    const std::string path = "entries[" + std::to_string(i) + "]";
    const Object *o = (*arr)[i].as_object();
    if (o == nullptr) {
      r.error = path + ": expected an object";
      return r;
    }
    CacheEntry e;
    if (!ParseEntry(*o, path, e, r.error)) return r;
    cache.entries.push_back(std::move(e));
  }
  r.cache = std::move(cache);
  return r;
}

std::string SerializeTuningCache(const TuningCache &cache) {
  json::Array entries;
  entries.reserve(cache.entries.size());
  for (const CacheEntry &e : cache.entries) entries.push_back(detail::EntryJson(e));
  return json::Serialize(Value(Object{{"version", cache.version}, {"entries", Value(std::move(entries))}}));
}

// ---- AmdTuningDb ---------------------------------------------------------------

bool AmdTuningDb::Put(CacheEntry entry) {
  if (entry.gpu.empty()) return false;
  Key key{entry.gpu, entry.op, entry.shape.m, entry.shape.n, entry.shape.k, entry.shape.dtype};
  entries_[std::move(key)] = std::move(entry);
  return true;
}

std::optional<CacheEntry> AmdTuningDb::Get(std::string_view gpu, std::string_view op, const Shape &s) const {
  const auto it = entries_.find(Key{std::string(gpu), std::string(op), s.m, s.n, s.k, s.dtype});
  if (it == entries_.end()) return std::nullopt;
  return it->second;
}

std::vector<CacheEntry> AmdTuningDb::Entries(std::string_view gpu) const {
  std::vector<CacheEntry> out;
  for (const auto &kv : entries_)
    if (kv.first.gpu == gpu) out.push_back(kv.second);
  return out;
}

std::vector<std::string> AmdTuningDb::Namespaces() const {
  std::vector<std::string> out;
  for (const auto &kv : entries_)
    if (out.empty() || out.back() != kv.first.gpu) out.push_back(kv.first.gpu);
  return out;
}

std::string AmdTuningDb::Serialize() const {
  TuningCache c;
  for (const auto &kv : entries_) c.entries.push_back(kv.second);
  return SerializeTuningCache(c);
}

std::string AmdTuningDb::SerializeNamespace(std::string_view gpu) const {
  TuningCache c;
  c.entries = Entries(gpu);
  return SerializeTuningCache(c);
}

AmdTuningDbParseResult AmdTuningDb::Parse(std::string_view text) {
  AmdTuningDbParseResult r;
  TuningCacheParseResult p = ParseTuningCache(text);
  if (!p.ok()) {
    r.error = std::move(p.error);
    return r;
  }
  AmdTuningDb db;
  for (size_t i = 0; i < p.cache->entries.size(); ++i) {
    if (!db.Put(p.cache->entries[i])) {
      r.error = "entries[" + std::to_string(i) +
                "].gpu: empty gpu - a tuning entry must belong to a namespace (e.g. gfx950)";
      return r;
    }
  }
  r.db = std::move(db);
  return r;
}

// ---- gate -------------------------------------------------------------------------

bool PassesCorrectnessGate(const Correctness &c, double ceiling) {
  return c.cosine >= kGateCosineThreshold && c.pcc >= kGatePccThreshold && c.max_rel_err <= ceiling;
}

double RelCeiling(std::string_view op, std::int64_t k) {
  if (k < 256 && op.substr(0, 6) != "fused_") return kGateMaxRelErrStrict;
  return INFINITY;
}

std::optional<std::size_t> SelectBestValidated(const std::vector<VariantResult> &results) {
  std::optional<std::size_t> best;
  for (std::size_t i = 0; i < results.size(); ++i) {
    if (!results[i].validated || !results[i].time_ms) continue;
    if (!best || *results[i].time_ms < *results[*best].time_ms) best = i;
  }
  return best;
}

}  // namespace pk::autotune
