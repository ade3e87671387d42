// runtime_test.cpp -- C++ API tests of the runtime layer (no GPU needed).
//
// Built and run by tests/test_runtime_cpp.py against the in-tree library, as
// a C++ caller would link it.  Mirrors cases of the reference's gtests
// (lib/Runtime/tests/runtime_test.cpp, kernel_cache_persist_test.cpp,
// device_detect_test.cpp; lib/Autotune/tests/amd_tuning_db_test.cpp) in a
// minimal self-contained harness.
#include <cstdio>
#include <cstdlib>
#include <filesystem>
#include <fstream>
#include <string>

#include "polykernel_amd_runtime.hpp"

namespace {

int g_failures = 0, g_checks = 0;

#define CHECK(cond)                                                          \
  do {                                                                       \
    ++g_checks;                                                              \
    if (!(cond)) {                                                           \
      ++g_failures;                                                          \
      std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond); \
    }                                                                        \
  } while (0)

#define CHECK_CONTAINS(haystack, needle)                                                     \
  do {                                                                                       \
    ++g_checks;                                                                              \
    if (std::string(haystack).find(needle) == std::string::npos) {                           \
      ++g_failures;                                                                          \
      std::fprintf(stderr, "%s:%d: '%s' not in '%s'\n", __FILE__, __LINE__, needle,          \
                   std::string(haystack).c_str());                                           \
    }                                                                                        \
  } while (0)

using namespace pk;
using autotune::CacheEntry;
using autotune::Config;
using autotune::Shape;

const Shape kShape{2048, 4096, 11008, "bf16"};
const char *kOp = "fused_matmul_bias_gelu";
const Config kBest950{256, 256, 32, 4, 8, 2, 5};
const Config kBest942{128, 128, 64, 4, 8, 4, 2};

CacheEntry Entry(std::string gpu, Config best, bool validated = true) {
  CacheEntry e;
  e.gpu = std::move(gpu);
  e.op = kOp;
  e.shape = kShape;
  e.best = best;
  e.scored_by = "measure";
  e.time_ms = 0.5;
  e.validated = validated;
  e.correctness = {0.99999, 1e-3, 0.9999};
  return e;
}

void TestDeviceDetect() {
  CHECK(runtime::ParseGcnArchName("gfx950:sramecc+:xnack-") == "gfx950");
  CHECK(runtime::ParseGcnArchName("gfx950") == "gfx950");
  CHECK(runtime::ParseGcnArchName("gfx90a:xnack+") == "gfx90a");
  CHECK(runtime::ParseGcnArchName("amdgcn-amd-amdhsa--gfx942:sramecc+") == "gfx942");
  CHECK(runtime::ParseGcnArchName("").empty());
  CHECK(runtime::ParseGcnArchName("gfx").empty());
  CHECK(runtime::ParseGcnArchName("gfxabc").empty());
  CHECK(runtime::ParseGcnArchName("sm_90").empty());
  runtime::FixedArchDetector det("gfx950", "mock");
  CHECK(det.Detect(0) == (runtime::DeviceInfo{"gfx950", "mock"}));
  CHECK(det.Detect(3) == det.Detect(0));  // ordinal-independent
  runtime::HipDeviceDetector hip;         // constructible and callable without a GPU
  (void)hip.Detect(0);
}

void TestTuningDb() {
  autotune::AmdTuningDb db;
  CHECK(db.Put(Entry("gfx950", kBest950)));
  CHECK(db.Put(Entry("gfx942", kBest942)));
  CHECK(!db.Put(Entry("", kBest942)));
  CHECK(db.Namespaces() == (std::vector<std::string>{"gfx942", "gfx950"}));
  CHECK(db.Get("gfx950", kOp, kShape)->best == kBest950);
  CHECK(!db.Get("gfx900", kOp, kShape));
  const std::string only950 = db.SerializeNamespace("gfx950");
  CHECK_CONTAINS(only950, "\"gpu\":\"gfx950\"");
  CHECK(only950.find("gfx942") == std::string::npos);
  auto back = autotune::AmdTuningDb::Parse(db.Serialize());
  CHECK(back.ok());
  CHECK(back.ok() && back.db->Size() == 2 && back.db->Get("gfx942", kOp, kShape) == db.Get("gfx942", kOp, kShape));
  // strings survive escapes, \u sequences and surrogate pairs
  auto p = autotune::ParseTuningCache(
      R"({"version":1,"entries":[{"gpu":"gfx950","op":"q\"\\\/é😀","shape":{"M":1,"N":2,"K":3,"dtype":"bf16"},)"
      R"("best":{"block_m":1,"block_n":1,"block_k":1,"num_warps":1,"vector_width":1,"unroll":1,"shared_memory_stages":1},)"
      R"("scored_by":"measure","time_ms":1e-3,"validated":true,"correctness":{"cosine":1,"max_rel_err":0,"pcc":1}}]})");
  CHECK(p.ok());
  if (p.ok()) {
    CHECK(p.cache->entries[0].op == "q\"\\/\xc3\xa9\xf0\x9f\x98\x80");
    auto again = autotune::ParseTuningCache(autotune::SerializeTuningCache(*p.cache));
    CHECK(again.ok() && *again.cache == *p.cache);
  }
  CHECK(!autotune::ParseTuningCache(R"({"version":1,"entries":[],"x":"\ud83d"})").ok());  // lone surrogate
  CHECK(!autotune::ParseTuningCache("{\"version\":1,\"entries\":[],\"x\":\"\xff\"}").ok());  // bad UTF-8
  CHECK(!autotune::ParseTuningCache(R"({"version":01,"entries":[]})").ok());               // leading zero
  std::string deep(2000, '[');
  CHECK_CONTAINS(autotune::ParseTuningCache(deep).error, "malformed JSON");  // bounded depth, no crash
}

void TestSelectPerGpu() {
  runtime::KernelCache cache;
  CHECK(cache.Put(Entry("gfx950", kBest950)));
  CHECK(cache.Put(Entry("gfx942", kBest942)));
  const auto res = cache.SelectPerGpu({"gfx950", "gfx942", "gfx900"}, kOp, kShape);
  CHECK(res.size() == 3);
  CHECK(res[0].second.ok() && res[0].second.entry->best == kBest950);
  CHECK(res[1].second.ok() && res[1].second.entry->best == kBest942);
  CHECK(!res[2].second.ok());
  CHECK(res[2].second.error ==
        "no tuned kernel for gfx900/fused_matmul_bias_gelu/M=2048,N=4096,K=11008,bf16; run the autotuner "
        "(polykernel_amd.autotune) to populate the cache");
}

void TestRuntime() {
  runtime::KernelCache cache;
  cache.Put(Entry("gfx950", kBest950));
  cache.Put(Entry("gfx942", kBest942, /*validated=*/false));
  runtime::FixedArchDetector det950("gfx950"), det942("gfx942");

  runtime::Runtime rt(det950, cache);
  std::string err;
  CHECK(!rt.Run(kOp, kShape, nullptr, err));
  CHECK_CONTAINS(err, "no compiled launcher registered");

  int served = 0;
  Config seen{};
  rt.RegisterLauncher(kOp, [&](const CacheEntry &e, void *io, std::string &) {
    ++served;
    seen = e.best;
    *static_cast<int *>(io) = 42;
    return true;
  });
  int io = 0;
  err.clear();
  CHECK(rt.Run(kOp, kShape, &io, err) && err.empty());
  CHECK(served == 1 && io == 42 && seen == kBest950);

  // a miss never reaches the launcher
  CHECK(!rt.Run(kOp, Shape{128, 128, 128, "bf16"}, &io, err));
  CHECK_CONTAINS(err, "no tuned kernel");
  CHECK_CONTAINS(err, "M=128,N=128,K=128");
  CHECK(served == 1);

  runtime::Runtime rt942(det942, cache);
  rt942.RegisterLauncher(kOp, [&](const CacheEntry &, void *, std::string &) { return ++served, true; });
  CHECK(!rt942.Run(kOp, kShape, &io, err));
  CHECK_CONTAINS(err, "not validated");
  CHECK(served == 1);

  // a launch failure comes back with the launcher's message
  rt.RegisterLauncher(kOp, [](const CacheEntry &, void *, std::string &e) {
    e = "hip launch failed: invalid configuration";
    return false;
  });
  CHECK(!rt.Run(kOp, kShape, &io, err));
  CHECK_CONTAINS(err, "hip launch failed");

  // the built-in launchers refuse a foreign config before any device call
  runtime::KernelCache c2;
  CacheEntry odd = Entry("gfx950", Config{96, 96, 32, 4, 8, 2, 5});
  c2.Put(odd);
  runtime::Runtime rt2(det950, c2);
  runtime::RegisterBuiltinLaunchers(rt2);
  CHECK(rt2.HasLauncher("matmul_int8_residual") && rt2.HasLauncher("fused_kv_append_attention"));
  runtime::MatmulIO mio{};
  mio.M = 2048;
  mio.N = 4096;
  mio.K = 11008;
  CHECK(!rt2.Run(kOp, kShape, &mio, err));
  CHECK_CONTAINS(err, "is not one the gfx950 kernels implement");
  CHECK(!rt2.Run(kOp, kShape, nullptr, err));
  CHECK_CONTAINS(err, "null argument block");
}

void TestConfigSpace() {
  const Shape g{4096, 16384, 4096, "bf16"};
  const auto all = autotune::ConfigSpace::Candidates("fused_matmul_bias_gelu", g);
  CHECK(all.size() >= 5);
  for (const Config &c : all) CHECK(autotune::ConfigSpace::IsAdmissible("fused_matmul_bias_gelu", g, c));
  CHECK(autotune::ConfigSpace::LdsBytes("matmul", g, all[0]) == 160 * 1024);  // 5-stage ring fills the CU
  // a 64 KiB budget keeps only the small tiles
  autotune::ArchLimits small;
  small.lds_per_cu_bytes = 64 * 1024;
  const auto pruned = autotune::ConfigSpace::Candidates("fused_matmul_bias_gelu", g, small);
  CHECK(!pruned.empty() && pruned.size() < all.size());
  for (const Config &c : pruned) CHECK(c.block_m <= 128);
  CHECK_CONTAINS(autotune::ConfigSpace::RejectionReason("matmul", g, all[0], small), "LDS");
  CHECK_CONTAINS(autotune::ConfigSpace::RejectionReason("matmul", g, Config{256, 256, 32, 32, 8, 2, 5}),
                 "max_threads_per_workgroup");
  CHECK(autotune::ConfigSpace::RejectionReason("conv", g, all[0]) == "unknown op");
  const auto d = autotune::ConfigSpace::Default("fused_matmul_bias_gelu", g);
  CHECK(d && *d == all[0]);
  const Shape q{16, 28672, 8192, "int8"};
  const auto i8 = autotune::ConfigSpace::Candidates("matmul_int8_gelu", q);
  CHECK(i8.size() > 50);
  const auto di8 = autotune::ConfigSpace::Default("matmul_int8_gelu", q);
  CHECK(di8 && std::find(i8.begin(), i8.end(), *di8) != i8.end());
  CHECK(autotune::ConfigSpace::Candidates("matmul_int8_gelu", Shape{16, 28672, 8192, "bf16"}).empty());
  CHECK(autotune::BuiltinOps().size() == 10);
  CHECK(autotune::OpShape("fused_softmax_mask", 4, 8, 0).dtype == "fp32");
}

void TestCodeObjectRefusesChangedFile() {
  const std::filesystem::path dir = std::filesystem::temp_directory_path() / "pk_runtime_test";
  std::filesystem::create_directories(dir);
  const std::string path = (dir / "k.hsaco").string();
  {
    std::ofstream(path, std::ios::binary) << "not-a-code-object";
  }
  std::string hash, err;
  CHECK(runtime::HashFile(path, hash, err));
  runtime::CodeObject co;
  CHECK(!co.Load(runtime::CachedBinary{path, "0000000000000000"}, err));
  CHECK_CONTAINS(err, "changed since it was cached");
  CHECK(!co.loaded());
  CHECK(!co.Load(runtime::CachedBinary{(dir / "missing.hsaco").string(), hash}, err));
  CHECK_CONTAINS(err, "cannot read binary");
  CHECK(co.Function("k", err) == nullptr);
  CHECK_CONTAINS(err, "not loaded");
  std::filesystem::remove_all(dir);
}

void TestGate() {
  using autotune::Correctness;
  CHECK(autotune::PassesCorrectnessGate(Correctness{0.999, 0.01, 0.99}));
  CHECK(!autotune::PassesCorrectnessGate(Correctness{0.999, 0.0101, 0.99}));
  CHECK(autotune::PassesCorrectnessGate(Correctness{0.999, 0.05, 0.99}, autotune::kGateMaxRelErrLargeK));
  std::vector<autotune::VariantResult> v(3);
  v[0].validated = true;
  v[0].time_ms = 2.0;
  v[1].time_ms = 1.0;  // faster but not validated
  v[2].validated = true;
  v[2].time_ms = 2.0;
  CHECK(autotune::SelectBestValidated(v) == std::optional<size_t>(0));
}

}  // namespace

int main() {
  TestDeviceDetect();
  TestTuningDb();
  TestSelectPerGpu();
  TestRuntime();
  TestConfigSpace();
  TestCodeObjectRefusesChangedFile();
  TestGate();
  std::printf("%d checks, %d failures\n", g_checks, g_failures);
  if (g_failures == 0) std::printf("ALL PASSED\n");
  return g_failures == 0 ? 0 : 1;
}
