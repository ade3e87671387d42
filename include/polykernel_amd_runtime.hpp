// polykernel_amd_runtime.hpp -- C++ runtime of the gfx950 kernel library:
// tuning cache, kernel cache, device detection, detect -> select -> serve,
// correctness-gated autotuning and code-object loading.
//
// The class and function names, argument meanings and error strings follow
// the reference's runtime so that its callers port unchanged:
//   autotune::Config / Shape / Correctness / CacheEntry / TuningCache
//       include/PolyKernel/Autotune/ConfigSpace.h:24-40, TuningCache.h:46-107
//   autotune::ParseTuningCache / SerializeTuningCache   TuningCache.h:109-121
//   autotune::AmdTuningDb                                AmdTuningDb.h:40-123
//   autotune::PassesCorrectnessGate / SelectBestValidated  Benchmark.h:88-120
//   runtime::FormatKey / HashFile / KernelCache          KernelCache.h:38-157
//   runtime::DeviceDetector / ParseGcnArchName / HipDeviceDetector /
//       FixedArchDetector                                DeviceDetect.h:30-103
//   runtime::Runtime / LaunchFn / ResolveResult          Runtime.h:40-97
// What is MI355X-specific: the config space is the set of variants the gfx950
// kernels implement (waves of 64 lanes, 160 KiB of LDS per CU), the gate's
// golden is computed by naive device kernels, and tuned variants can be
// emitted as standalone code objects (.hsaco) that the runtime loads with
// hipModuleLoad after checking their FNV-1a hash.
#pragma once

#include <compare>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <map>
#include <optional>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

#include "polykernel_amd.h"
#include "polykernel_amd_runtime.h"

namespace pk::autotune {

inline constexpr int kTuningCacheVersion = 1;

// One point of the tuning space; field names are those of the tuning-cache
// schema (tuning/schema.json:65-79).  On gfx950 `num_warps` counts 64-lane
// waves per workgroup.
struct Config {
  int block_m = 0;
  int block_n = 0;
  int block_k = 0;
  int num_warps = 0;
  int vector_width = 0;
  int unroll = 0;
  int shared_memory_stages = 0;
  bool operator==(const Config &) const = default;
  std::strong_ordering operator<=>(const Config &) const = default;
};
PK_API std::string ToString(const Config &config);

struct Shape {
  std::int64_t m = 0;
  std::int64_t n = 0;
  std::int64_t k = 0;
  std::string dtype;
  bool operator==(const Shape &) const = default;
};

struct Correctness {
  double cosine = 0.0;
  double max_rel_err = 0.0;
  double pcc = 0.0;
  bool operator==(const Correctness &) const = default;
};

struct CacheEntry {
  std::string gpu;  // cache namespace, "gfx950" on MI355X
  std::string op;
  Shape shape;
  Config best;
  std::string scored_by;         // "measure" | "compile_time_model"
  std::optional<double> time_ms;  // nullopt <=> JSON null
  bool validated = false;
  Correctness correctness;
  bool operator==(const CacheEntry &) const = default;
};

struct TuningCache {
  int version = kTuningCacheVersion;
  std::vector<CacheEntry> entries;
  bool operator==(const TuningCache &) const = default;
};

struct TuningCacheParseResult {
  std::optional<TuningCache> cache;
  std::string error;  // field path + reason, e.g. "entries[0].scored_by: ..."
  bool ok() const { return cache.has_value(); }
};

// Strict: a missing or wrongly typed required field is an error naming its
// path; the version must be kTuningCacheVersion; time_ms may be null.
PK_API TuningCacheParseResult ParseTuningCache(std::string_view json);
PK_API std::string SerializeTuningCache(const TuningCache &cache);

struct AmdTuningDbParseResult;

// Tuning entries partitioned by gpu namespace; (gpu, op, shape) is the key.
class PK_API AmdTuningDb {
 public:
  // Last writer wins; false (no-op) for an empty gpu.
  bool Put(CacheEntry entry);
  std::optional<CacheEntry> Get(std::string_view gpu, std::string_view op, const Shape &shape) const;
  // One namespace's entries in (op, M, N, K, dtype) order.
  std::vector<CacheEntry> Entries(std::string_view gpu) const;
  std::vector<std::string> Namespaces() const;  // sorted
  std::size_t Size() const { return entries_.size(); }
  std::string Serialize() const;
  std::string SerializeNamespace(std::string_view gpu) const;
  static AmdTuningDbParseResult Parse(std::string_view json);

 private:
  struct Key {
    std::string gpu, op;
    std::int64_t m, n, k;
    std::string dtype;
    auto operator<=>(const Key &) const = default;
  };
  std::map<Key, CacheEntry> entries_;
};

struct AmdTuningDbParseResult {
  std::optional<AmdTuningDb> db;
  std::string error;
  bool ok() const { return db.has_value(); }
};

// ---- correctness gate -----------------------------------------------------
inline constexpr double kGateCosineThreshold = 0.999;
inline constexpr double kGatePccThreshold = 0.99;
inline constexpr double kGateMaxRelErrStrict = 1e-2;
inline constexpr double kGateMaxRelErrLargeK = 5e-2;

// cosine >= 0.999 && pcc >= 0.99 && max_rel_err <= ceiling.
PK_API bool PassesCorrectnessGate(const Correctness &c, double max_rel_ceiling = kGateMaxRelErrStrict);
// The max_rel_err ceiling the autotuner applies: strict 1e-2 for unfused ops
// with K < 256, no bound otherwise (near-zero outputs of long reductions make
// the relative error meaningless there; cosine and pcc still gate).
// Follows tools/polykernel-bench/bench.py:297-306 of the reference.
PK_API double RelCeiling(std::string_view op, std::int64_t k);

struct VariantResult {
  std::string name;
  Correctness correctness;
  bool validated = false;
  std::optional<double> time_ms;  // nullopt <=> failed the gate, never timed
  // GEMM-class ops: outputs outside the fp32 error model (pk_gate_matmul*);
  // a validated variant has none.  nullopt for ops gated on the metrics only.
  std::optional<unsigned long long> model_violations;
  bool operator==(const VariantResult &) const = default;
};
// Fastest validated variant; ties go to the lowest index; nullopt if none.
PK_API std::optional<std::size_t> SelectBestValidated(const std::vector<VariantResult> &results);

// ---- gfx950 config space ----------------------------------------------------
struct ArchLimits {
  long long lds_per_cu_bytes = 160 * 1024;
  int wave_size = 64;
  int max_threads_per_workgroup = 1024;
  int vgprs_per_lane = 512;  // 256 arch VGPRs + 256 AccVGPRs
  int num_cus = 256;
};

class PK_API ConfigSpace {
 public:
  // Every configuration the gfx950 kernels implement for (op, shape), in the
  // library's order of preference, pruned by `limits`.  Empty for an unknown
  // op or a shape no variant accepts.
  static std::vector<Config> Candidates(std::string_view op, const Shape &shape,
                                        const ArchLimits &limits = {});
  // The configuration the library's own heuristic picks (what the plain
  // launch_* entry points run); nullopt if the op or shape is unsupported.
  static std::optional<Config> Default(std::string_view op, const Shape &shape);
  // "" when admissible, else the violated rule.
  static std::string RejectionReason(std::string_view op, const Shape &shape, const Config &config,
                                     const ArchLimits &limits = {});
  static bool IsAdmissible(std::string_view op, const Shape &shape, const Config &config,
                           const ArchLimits &limits = {}) {
    return RejectionReason(op, shape, config, limits).empty();
  }
  // LDS bytes one workgroup of `config` allocates at `shape` (0 for unknown ops).
  static long long LdsBytes(std::string_view op, const Shape &shape, const Config &config);
};

// The ops the runtime serves, with the shape key each one uses:
//   matmul, fused_matmul_bias_gelu, fused_matmul_bias_residual
//       {M, N, K, "bf16"}
//   matmul_int8, matmul_int8_gelu, matmul_int8_residual   {M, N, K, "int8"}
//   fused_rmsnorm_matmul                                  {M, N, K, "bf16"}
//   fused_residual_rmsnorm                       {rows, cols, 0, "bf16"}
//   fused_softmax_mask                           {rows, cols, 0, "fp32"}
//   fused_kv_append_attention                  {S_q, S_cache + S_q, D, "bf16"}
PK_API const std::vector<std::string> &BuiltinOps();
PK_API Shape OpShape(std::string_view op, std::int64_t m, std::int64_t n, std::int64_t k);

// ---- autotuner ---------------------------------------------------------------
class PK_API HipEventTimer {
 public:
  HipEventTimer();
  ~HipEventTimer();
  HipEventTimer(const HipEventTimer &) = delete;
  HipEventTimer &operator=(const HipEventTimer &) = delete;
  bool ok() const { return start_ != nullptr && stop_ != nullptr; }
  void Start(void *stream);
  void Stop(void *stream);
  // Synchronises on the stop event; negative on a HIP error.
  float ElapsedMs();

 private:
  void *start_ = nullptr;
  void *stop_ = nullptr;
};

struct AutotuneOptions {
  int warmup = 3;
  int iters = 20;
  // the timed launches of all gated variants are spread over this many
  // interleaved passes (median over all samples of a variant)
  int rounds = 5;
  // HBM-bound ops (int8, row-wise, softmax) are timed over rotating copies of
  // their inputs whose total reaches this many bytes (at most 4 copies), so
  // the 256 MiB MALL does not serve them; MFMA-bound ops use one copy.
  std::size_t rotate_bytes = std::size_t(600) << 20;
  std::optional<double> rel_ceiling;   // default RelCeiling(op, K)
  std::optional<std::size_t> max_variants;  // sweep only the first N candidates
  std::uint64_t seed = 0xC0FFEE;
  int batch_heads = 32;  // B*H for fused_kv_append_attention
  bool verbose = false;
  // Test hook (tools/polykernel-bench/bench.py --inject-broken of the
  // reference): add one fast-but-wrong variant, named "broken_fast ...", that
  // the gate must reject -- GEMM-class ops only.
  bool inject_broken = false;
};

struct AutotuneResult {
  CacheEntry entry;  // validated == false when no variant passed the gate
  std::vector<std::pair<Config, VariantResult>> variants;
};

// Sweep the candidates of (op, shape) on the current device: every variant is
// first compared with a naive device reference of the op on seeded inputs
// (cosine / max_rel_err / pcc; GEMM-class ops also the fp32 error model of
// pk_gate_matmul*); only variants that pass the gate are timed
// (HIP events, median of `iters`); the fastest validated one becomes the
// entry.  Returns false with `error` when the sweep could not run.
PK_API bool Autotune(std::string_view op, const Shape &shape, const AutotuneOptions &options,
                     AutotuneResult &result, std::string &error);

}  // namespace pk::autotune

namespace pk::runtime {

using autotune::CacheEntry;
using autotune::Config;
using autotune::Shape;

// "gpu/op/M=..,N=..,K=..,dtype" (lib/Runtime/KernelCache.cpp:36-42).
PK_API std::string FormatKey(std::string_view gpu, std::string_view op, const Shape &shape);

struct SelectionResult {
  std::optional<CacheEntry> entry;
  std::string error;
  bool ok() const { return entry.has_value(); }
};

struct CachedBinary {
  std::string so_path;      // the code object (.hsaco) or shared library on disk
  std::string kernel_hash;  // FNV-1a 64 of its bytes, 16 lower-case hex digits
  bool operator==(const CachedBinary &) const = default;
};

// FNV-1a 64-bit over the file's bytes (lib/Runtime/KernelCache.cpp:46-69).
PK_API bool HashFile(std::string_view path, std::string &hash_out, std::string &error);

class PK_API KernelCache {
 public:
  bool LoadTuningCache(std::string_view json, std::string &error);
  bool Put(CacheEntry entry);
  // Miss and unvalidated entries are errors, never a served entry.
  SelectionResult Select(std::string_view gpu, std::string_view op, const Shape &shape) const;
  std::size_t Size() const { return db_.Size(); }
  const autotune::AmdTuningDb &Db() const { return db_; }

  // A binary must back a present tuning entry.
  bool PutBinary(std::string_view gpu, std::string_view op, const Shape &shape, CachedBinary binary);
  std::optional<CachedBinary> GetBinary(std::string_view gpu, std::string_view op, const Shape &shape) const;

  // <dir>/tuning_db.json + <dir>/binaries.json; LoadPersisted leaves the
  // cache unchanged on any error.
  bool Persist(std::string_view cache_dir, std::string &error) const;
  bool LoadPersisted(std::string_view cache_dir, std::string &error);
  // Drops every entry whose binary is missing or whose hash changed; returns
  // how many were dropped.
  std::size_t InvalidateStale();
  std::vector<std::pair<std::string, SelectionResult>> SelectPerGpu(const std::vector<std::string> &gpus,
                                                                    std::string_view op,
                                                                    const Shape &shape) const;

 private:
  autotune::AmdTuningDb db_;
  std::map<std::string, CachedBinary> binaries_;
};

struct DeviceInfo {
  std::string arch;  // bare gfx token, e.g. "gfx950"
  std::string name;
  bool operator==(const DeviceInfo &) const = default;
};

class PK_API DeviceDetector {
 public:
  virtual ~DeviceDetector() = default;
  virtual std::optional<DeviceInfo> Detect(int ordinal = 0) const = 0;
};

// "gfx950:sramecc+:xnack-" -> "gfx950"; "" when no gfx<digit> token.
PK_API std::string ParseGcnArchName(std::string_view gcn_arch_name);

// hipGetDeviceProperties of `ordinal`, queried once per process and ordinal.
class PK_API HipDeviceDetector final : public DeviceDetector {
 public:
  std::optional<DeviceInfo> Detect(int ordinal = 0) const override;

 private:
  static std::optional<DeviceInfo> Query(int ordinal);
};

class PK_API FixedArchDetector final : public DeviceDetector {
 public:
  explicit FixedArchDetector(std::string arch, std::string name = "mock-device")
      : arch_(std::move(arch)), name_(std::move(name)) {}
  std::optional<DeviceInfo> Detect(int ordinal = 0) const override;

 private:
  std::string arch_, name_;
};

using LaunchFn = std::function<bool(const CacheEntry &entry, void *io, std::string &error)>;

struct ResolveResult {
  std::optional<DeviceInfo> device;
  std::optional<CacheEntry> entry;
  std::string error;
  bool ok() const { return entry.has_value(); }
};

class PK_API Runtime {
 public:
  Runtime(const DeviceDetector &detector, const KernelCache &cache) : detector_(detector), cache_(cache) {}
  void RegisterLauncher(std::string op, LaunchFn fn) { launchers_[std::move(op)] = std::move(fn); }
  bool HasLauncher(std::string_view op) const { return launchers_.find(op) != launchers_.end(); }
  // detect + select.
  ResolveResult Resolve(std::string_view op, const Shape &shape) const;
  // detect + select + serve with the registered launcher.
  bool Run(std::string_view op, const Shape &shape, void *io, std::string &error);

 private:
  const DeviceDetector &detector_;
  const KernelCache &cache_;
  std::map<std::string, LaunchFn, std::less<>> launchers_;
};

// ---- argument blocks (`io`) of the built-in launchers -------------------------
// The C structs of polykernel_amd_runtime.h, shared with C and ctypes callers.
using MatmulIO = pk_matmul_io;
using MatmulInt8IO = pk_matmul_int8_io;
using RmsnormMatmulIO = pk_rmsnorm_matmul_io;
using ResidualRmsnormIO = pk_residual_rmsnorm_io;
using SoftmaxMaskIO = pk_softmax_mask_io;
using KvAppendAttentionIO = pk_kv_append_attention_io;

// Register a launcher for every op of BuiltinOps(): each checks that the io
// block's dimensions are the selected entry's shape and that the entry's
// config is one the kernels implement, then launches through the C-ABI.
PK_API void RegisterBuiltinLaunchers(Runtime &runtime);

// Serve every built-in op (the GEMM family, fused_rmsnorm_matmul,
// fused_residual_rmsnorm, fused_softmax_mask, fused_kv_append_attention and
// the three int8 ops) from the code objects `cache` holds for their entries
// (codegen::EmitCodeObject): the object is loaded once (hash-checked) and
// launched with hipModuleLaunchKernel, with the linked path's launch
// geometry and operand checks for the entry's config.  An entry without a
// cached code object is an error.  `cache` must outlive the runtime.
PK_API void RegisterCodeObjectLaunchers(Runtime &runtime, const KernelCache &cache);

// ---- code objects -------------------------------------------------------------
// A code object loaded with hipModuleLoad (the binary half of a cache entry).
class PK_API CodeObject {
 public:
  CodeObject() = default;
  ~CodeObject();
  CodeObject(CodeObject &&o) noexcept;
  CodeObject &operator=(CodeObject &&o) noexcept;
  CodeObject(const CodeObject &) = delete;
  CodeObject &operator=(const CodeObject &) = delete;

  // Loads `binary.so_path` after checking its FNV-1a hash equals
  // `binary.kernel_hash` (a changed or missing file is refused).
  bool Load(const CachedBinary &binary, std::string &error);
  // hipFunction_t of `name` as void*, or nullptr with `error`.
  void *Function(std::string_view name, std::string &error) const;
  bool loaded() const { return module_ != nullptr; }

 private:
  void *module_ = nullptr;
};

}  // namespace pk::runtime

namespace pk::codegen {

// The gfx950 HIP source of a tuned entry: the op's kernel template
// instantiated at the entry's config behind fixed extern "C" entry points
// (pk_gemm; pk_row / pk_row_any; pk_panel; pk_fa_fused / pk_fa_combine or
// pk_att / pk_att_unaligned / pk_att_combine / pk_kv_append; pk_int8_stream /
// pk_int8_reduce).  An op outside the tuning cache's ops, or a config the
// kernels do not implement for the shape, is refused.
PK_API bool EmitSource(const autotune::CacheEntry &entry, std::string &source, std::string &error);
// hipcc --genco for gfx950 (the library's flags) in a child process; the
// kernel headers are found under csrc_dir.
PK_API bool CompileCodeObject(const std::string &source_path, const std::string &csrc_dir,
                              const std::string &out_path, std::string &error);
// Emit + compile into out_dir, then record the entry and its code object
// (absolute path, FNV-1a hash) in `cache`.
PK_API bool EmitCodeObject(runtime::KernelCache &cache, const autotune::CacheEntry &entry,
                           const std::string &csrc_dir, const std::string &out_dir, std::string &error);

}  // namespace pk::codegen
