// capi.cpp -- C-ABI over the runtime (include/polykernel_amd_runtime.h).
#include <cmath>
#include <cstring>
#include <memory>

#include "internal.hpp"

namespace {

thread_local std::string g_text;

using pk::autotune::CacheEntry;
using pk::autotune::Shape;

int Text(std::string s) {
  g_text = std::move(s);
  return PK_OK;
}

int Fail(int code, const std::string &msg) {
  pk::set_error("%s", msg.c_str());
  return code;
}

Shape MakeShape(long long M, long long N, long long K, const char *dtype) {
  return Shape{M, N, K, dtype ? dtype : ""};
}

std::string Str(const char *s) { return s ? s : ""; }

}  // namespace

struct pk_kernel_cache {
  pk::runtime::KernelCache cache;
};

struct pk_runtime {
  std::unique_ptr<pk::runtime::DeviceDetector> detector;
  pk::runtime::Runtime rt;
  pk_runtime(std::unique_ptr<pk::runtime::DeviceDetector> d, const pk::runtime::KernelCache &c)
      : detector(std::move(d)), rt(*detector, c) {}
};

extern "C" {

PK_API const char *pk_last_text(void) { return g_text.c_str(); }

PK_API pk_kernel_cache *pk_cache_create(void) { return new (std::nothrow) pk_kernel_cache(); }

PK_API void pk_cache_destroy(pk_kernel_cache *c) { delete c; }

PK_API int pk_cache_load_tuning(pk_kernel_cache *c, const char *json) {
  if (!c || !json) return Fail(PK_ERR_INVALID_ARG, "pk_cache_load_tuning: null argument");
  std::string err;
  if (!c->cache.LoadTuningCache(json, err)) return Fail(PK_ERR_INVALID_ARG, err);
  return PK_OK;
}

PK_API int pk_cache_put(pk_kernel_cache *c, const char *entry_json) {
  if (!c || !entry_json) return Fail(PK_ERR_INVALID_ARG, "pk_cache_put: null argument");
  const std::string doc = std::string("{\"version\":1,\"entries\":[") + entry_json + "]}";
  pk::autotune::TuningCacheParseResult p = pk::autotune::ParseTuningCache(doc);
  if (!p.ok()) return Fail(PK_ERR_INVALID_ARG, "pk_cache_put: " + p.error);
  if (!c->cache.Put(p.cache->entries.at(0))) return Fail(PK_ERR_INVALID_ARG, "pk_cache_put: empty gpu");
  return PK_OK;
}

PK_API long long pk_cache_size(const pk_kernel_cache *c) { return c ? (long long)c->cache.Size() : 0; }

PK_API int pk_cache_serialize(const pk_kernel_cache *c) {
  if (!c) return Fail(PK_ERR_INVALID_ARG, "pk_cache_serialize: null cache");
  return Text(c->cache.Db().Serialize());
}

PK_API int pk_cache_select(const pk_kernel_cache *c, const char *gpu, const char *op, long long M, long long N,
                           long long K, const char *dtype) {
  if (!c || !gpu || !op || !dtype) return Fail(PK_ERR_INVALID_ARG, "pk_cache_select: null argument");
  pk::runtime::SelectionResult r = c->cache.Select(gpu, op, MakeShape(M, N, K, dtype));
  if (!r.ok()) return Fail(PK_ERR_NOT_FOUND, r.error);
  return Text(pk::json::Serialize(pk::autotune::detail::EntryJson(*r.entry)));
}

PK_API int pk_cache_put_binary(pk_kernel_cache *c, const char *gpu, const char *op, long long M, long long N,
                               long long K, const char *dtype, const char *so_path, const char *hash) {
  if (!c || !gpu || !op || !dtype || !so_path || !hash)
    return Fail(PK_ERR_INVALID_ARG, "pk_cache_put_binary: null argument");
  if (!c->cache.PutBinary(gpu, op, MakeShape(M, N, K, dtype), {so_path, hash}))
    return Fail(PK_ERR_NOT_FOUND, "pk_cache_put_binary: no tuning entry for " +
                                      pk::runtime::FormatKey(gpu, op, MakeShape(M, N, K, dtype)));
  return PK_OK;
}

PK_API int pk_cache_get_binary(const pk_kernel_cache *c, const char *gpu, const char *op, long long M, long long N,
                               long long K, const char *dtype) {
  if (!c || !gpu || !op || !dtype) return Fail(PK_ERR_INVALID_ARG, "pk_cache_get_binary: null argument");
  const auto b = c->cache.GetBinary(gpu, op, MakeShape(M, N, K, dtype));
  if (!b) return Fail(PK_ERR_NOT_FOUND, "no binary for " + pk::runtime::FormatKey(gpu, op, MakeShape(M, N, K, dtype)));
  return Text(pk::json::Serialize(pk::json::Object{{"so_path", b->so_path}, {"kernel_hash", b->kernel_hash}}));
}

PK_API int pk_cache_persist(const pk_kernel_cache *c, const char *dir) {
  if (!c || !dir) return Fail(PK_ERR_INVALID_ARG, "pk_cache_persist: null argument");
  std::string err;
  if (!c->cache.Persist(dir, err)) return Fail(PK_ERR_INVALID_ARG, err);
  return PK_OK;
}

PK_API int pk_cache_load_persisted(pk_kernel_cache *c, const char *dir) {
  if (!c || !dir) return Fail(PK_ERR_INVALID_ARG, "pk_cache_load_persisted: null argument");
  std::string err;
  if (!c->cache.LoadPersisted(dir, err)) return Fail(PK_ERR_INVALID_ARG, err);
  return PK_OK;
}

PK_API long long pk_cache_invalidate_stale(pk_kernel_cache *c) {
  return c ? (long long)c->cache.InvalidateStale() : 0;
}

PK_API int pk_hash_file(const char *path) {
  if (!path) return Fail(PK_ERR_INVALID_ARG, "pk_hash_file: null path");
  std::string h, err;
  if (!pk::runtime::HashFile(path, h, err)) return Fail(PK_ERR_INVALID_ARG, err);
  return Text(h);
}

PK_API int pk_format_key(const char *gpu, const char *op, long long M, long long N, long long K, const char *dtype) {
  return Text(pk::runtime::FormatKey(Str(gpu), Str(op), MakeShape(M, N, K, dtype)));
}

PK_API int pk_passes_correctness_gate(double cosine, double max_rel_err, double pcc, double ceiling) {
  return pk::autotune::PassesCorrectnessGate({cosine, max_rel_err, pcc}, ceiling) ? 1 : 0;
}

PK_API double pk_rel_ceiling(const char *op, long long K) { return pk::autotune::RelCeiling(Str(op), K); }

PK_API int pk_select_best_validated(const int *validated, const double *time_ms, int n) {
  if (n <= 0 || !validated || !time_ms) return -1;
  std::vector<pk::autotune::VariantResult> v(n);
  for (int i = 0; i < n; ++i) {
    v[i].validated = validated[i] != 0;
    if (!std::isnan(time_ms[i])) v[i].time_ms = time_ms[i];
  }
  const auto b = pk::autotune::SelectBestValidated(v);
  return b ? (int)*b : -1;
}

PK_API int pk_config_candidates(const char *op, long long M, long long N, long long K, const char *dtype) {
  if (!op || !dtype) return Fail(PK_ERR_INVALID_ARG, "pk_config_candidates: null argument");
  pk::json::Array arr;
  for (const auto &c : pk::autotune::ConfigSpace::Candidates(op, MakeShape(M, N, K, dtype)))
    arr.push_back(pk::autotune::detail::ConfigJson(c));
  return Text(pk::json::Serialize(pk::json::Value(std::move(arr))));
}

PK_API pk_runtime *pk_runtime_create_ex(const pk_kernel_cache *c, const char *fixed_arch, int flags) {
  if (!c) {
    pk::set_error("pk_runtime_create: null cache");
    return nullptr;
  }
  std::unique_ptr<pk::runtime::DeviceDetector> d;
  if (fixed_arch) d = std::make_unique<pk::runtime::FixedArchDetector>(fixed_arch);
  else d = std::make_unique<pk::runtime::HipDeviceDetector>();
  auto *rt = new (std::nothrow) pk_runtime(std::move(d), c->cache);
  if (!rt) return nullptr;
  pk::runtime::RegisterBuiltinLaunchers(rt->rt);
  if (flags & PK_RUNTIME_CODE_OBJECTS) pk::runtime::RegisterCodeObjectLaunchers(rt->rt, c->cache);
  return rt;
}

PK_API pk_runtime *pk_runtime_create(const pk_kernel_cache *c, const char *fixed_arch) {
  return pk_runtime_create_ex(c, fixed_arch, 0);
}

namespace {
bool ParseEntry(const char *entry_json, CacheEntry &e, std::string &error) {
  if (!entry_json) {
    error = "null entry";
    return false;
  }
  pk::autotune::TuningCacheParseResult p =
      pk::autotune::ParseTuningCache(std::string("{\"version\":1,\"entries\":[") + entry_json + "]}");
  if (!p.ok()) {
    error = p.error;
    return false;
  }
  e = p.cache->entries.at(0);
  return true;
}
}  // namespace

PK_API int pk_emit_source(const char *entry_json) {
  CacheEntry e;
  std::string err, src;
  if (!ParseEntry(entry_json, e, err)) return Fail(PK_ERR_INVALID_ARG, "pk_emit_source: " + err);
  if (!pk::codegen::EmitSource(e, src, err)) return Fail(PK_ERR_UNSUPPORTED, err);
  return Text(src);
}

PK_API int pk_emit_code_object(pk_kernel_cache *c, const char *entry_json, const char *csrc_dir,
                               const char *out_dir) {
  if (!c || !csrc_dir || !out_dir) return Fail(PK_ERR_INVALID_ARG, "pk_emit_code_object: null argument");
  CacheEntry e;
  std::string err;
  if (!ParseEntry(entry_json, e, err)) return Fail(PK_ERR_INVALID_ARG, "pk_emit_code_object: " + err);
  if (!pk::codegen::EmitCodeObject(c->cache, e, csrc_dir, out_dir, err)) return Fail(PK_ERR_UNSUPPORTED, err);
  return PK_OK;
}

PK_API void pk_runtime_destroy(pk_runtime *rt) { delete rt; }

PK_API int pk_runtime_resolve(pk_runtime *rt, const char *op, long long M, long long N, long long K,
                              const char *dtype) {
  if (!rt || !op || !dtype) return Fail(PK_ERR_INVALID_ARG, "pk_runtime_resolve: null argument");
  pk::runtime::ResolveResult r = rt->rt.Resolve(op, MakeShape(M, N, K, dtype));
  if (!r.ok()) return Fail(r.device ? PK_ERR_NOT_FOUND : PK_ERR_NO_DEVICE, r.error);
  return Text(pk::json::Serialize(pk::autotune::detail::EntryJson(*r.entry)));
}

PK_API int pk_runtime_run(pk_runtime *rt, const char *op, long long M, long long N, long long K, const char *dtype,
                          void *io) {
  if (!rt || !op || !dtype) return Fail(PK_ERR_INVALID_ARG, "pk_runtime_run: null argument");
  const Shape s = MakeShape(M, N, K, dtype);
  pk::runtime::ResolveResult r = rt->rt.Resolve(op, s);
  if (!r.ok()) return Fail(r.device ? PK_ERR_NOT_FOUND : PK_ERR_NO_DEVICE, r.error);
  std::string err;
  if (!rt->rt.Run(op, s, io, err)) return Fail(PK_ERR_LAUNCH, err);
  return PK_OK;
}

PK_API int pk_autotune(const char *op, long long M, long long N, long long K, const char *dtype,
                       const char *options_json) {
  if (!op || !dtype) return Fail(PK_ERR_INVALID_ARG, "pk_autotune: null argument");
  pk::autotune::AutotuneOptions o;
  if (options_json && *options_json) {
    pk::json::ParseResult p = pk::json::Parse(options_json);
    if (!p.ok() || !p.value->as_object()) return Fail(PK_ERR_INVALID_ARG, "pk_autotune: options must be an object");
    for (const auto &[k, v] : *p.value->as_object()) {
      const auto i = v.as_integer();
      const auto d = v.as_number();
      if (k == "warmup" && i) o.warmup = (int)*i;
      else if (k == "iters" && i) o.iters = (int)*i;
      else if (k == "rounds" && i && *i > 0) o.rounds = (int)*i;
      else if (k == "rotate_bytes" && i && *i >= 0) o.rotate_bytes = (size_t)*i;
      else if (k == "rel_ceiling" && d) o.rel_ceiling = *d;
      else if (k == "max_variants" && i && *i > 0) o.max_variants = (size_t)*i;
      else if (k == "seed" && i) o.seed = (uint64_t)*i;
      else if (k == "batch_heads" && i && *i > 0) o.batch_heads = (int)*i;
      else if (k == "verbose" && v.as_bool()) o.verbose = *v.as_bool();
      else if (k == "inject_broken" && v.as_bool()) o.inject_broken = *v.as_bool();
      else return Fail(PK_ERR_INVALID_ARG, "pk_autotune: bad option '" + k + "'");
    }
  }
  pk::autotune::AutotuneResult res;
  std::string err;
  if (!pk::autotune::Autotune(op, MakeShape(M, N, K, dtype), o, res, err)) return Fail(PK_ERR_LAUNCH, err);
  pk::json::Array vars;
  for (const auto &[cfg, v] : res.variants) {
    const pk::autotune::Correctness &c = v.correctness;
    vars.push_back(pk::json::Object{{"config", pk::autotune::detail::ConfigJson(cfg)},
                                    {"name", v.name},
                                    {"validated", v.validated},
                                    {"time_ms", v.time_ms ? pk::json::Value(*v.time_ms) : pk::json::Value()},
                                    {"model_violations", v.model_violations
                                                             ? pk::json::Value((long long)*v.model_violations)
                                                             : pk::json::Value()},
                                    {"correctness", pk::autotune::detail::CorrectnessJson(c)}});
  }
  return Text(pk::json::Serialize(pk::json::Object{{"entry", pk::autotune::detail::EntryJson(res.entry)},
                                                   {"variants", pk::json::Value(std::move(vars))}}));
}

}  // extern "C"
