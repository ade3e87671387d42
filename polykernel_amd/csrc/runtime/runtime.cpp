// runtime.cpp -- device detection, detect -> select -> serve, code objects.
//
// Resolve/Run follow lib/Runtime/Runtime.cpp:22-57 of the reference: a
// detection failure, a cache miss, an unvalidated entry, a missing launcher
// and a launch failure each come back as an error string, never a wrong
// kernel.  Detection maps hipDeviceProp_t::gcnArchName ("gfx950:sramecc+:
// xnack-") to its bare token like lib/Runtime/DeviceDetect.cpp:28-50.
#include <hip/hip_runtime_api.h>

#include <map>
#include <mutex>

#include "../../../include/polykernel_amd_runtime.hpp"

namespace pk::runtime {

std::string ParseGcnArchName(std::string_view s) {
  const size_t pos = s.find("gfx");
  if (pos == std::string_view::npos) return {};
  size_t end = pos + 3;
  if (end >= s.size() || s[end] < '0' || s[end] > '9') return {};
  while (end < s.size() && ((s[end] >= '0' && s[end] <= '9') || (s[end] >= 'a' && s[end] <= 'z'))) ++end;
  return std::string(s.substr(pos, end - pos));
}

// Device properties do not change while a process runs, and Runtime::Run
// detects on every call: the first answer per ordinal is kept.
std::optional<DeviceInfo> HipDeviceDetector::Detect(int ordinal) const {
  static std::mutex mu;
  static std::map<int, std::optional<DeviceInfo>> seen;
  {
    std::lock_guard<std::mutex> lock(mu);
    const auto it = seen.find(ordinal);
    if (it != seen.end()) return it->second;
  }
  std::optional<DeviceInfo> info = Query(ordinal);
  std::lock_guard<std::mutex> lock(mu);
  seen.emplace(ordinal, info);
  return info;
}

std::optional<DeviceInfo> HipDeviceDetector::Query(int ordinal) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || ordinal < 0 || ordinal >= count) {
    (void)hipGetLastError();
    return std::nullopt;
  }
  hipDeviceProp_t prop{};
  if (hipGetDeviceProperties(&prop, ordinal) != hipSuccess) {
    (void)hipGetLastError();
    return std::nullopt;
  }
  std::string arch = ParseGcnArchName(prop.gcnArchName);
  if (arch.empty()) return std::nullopt;
  return DeviceInfo{std::move(arch), prop.name};
}

std::optional<DeviceInfo> FixedArchDetector::Detect(int) const { return DeviceInfo{arch_, name_}; }

ResolveResult Runtime::Resolve(std::string_view op, const Shape &shape) const {
  ResolveResult r;
  std::optional<DeviceInfo> dev = detector_.Detect();
  if (!dev) {
    r.error = "device detection failed; no usable GPU to serve op " + std::string(op);
    return r;
  }
  r.device = dev;
  SelectionResult sel = cache_.Select(dev->arch, op, shape);
  if (!sel.ok()) {
    r.error = std::move(sel.error);
    return r;
  }
  r.entry = std::move(sel.entry);
  return r;
}

bool Runtime::Run(std::string_view op, const Shape &shape, void *io, std::string &error) {
  ResolveResult r = Resolve(op, shape);
  if (!r.ok()) {
    error = std::move(r.error);
    return false;
  }
  const auto it = launchers_.find(op);
  if (it == launchers_.end()) {
    error = "no compiled launcher registered for op " + std::string(op) +
            "; load the compiled variant (register its launch entry) first";
    return false;
  }
  return it->second(*r.entry, io, error);
}

// ---- code objects -------------------------------------------------------------

CodeObject::~CodeObject() {
  if (module_) (void)hipModuleUnload(static_cast<hipModule_t>(module_));
}

CodeObject::CodeObject(CodeObject &&o) noexcept : module_(o.module_) { o.module_ = nullptr; }

CodeObject &CodeObject::operator=(CodeObject &&o) noexcept {
  if (this != &o) {
    if (module_) (void)hipModuleUnload(static_cast<hipModule_t>(module_));
    module_ = o.module_;
    o.module_ = nullptr;
  }
  return *this;
}

bool CodeObject::Load(const CachedBinary &binary, std::string &error) {
  std::string hash;
  if (!HashFile(binary.so_path, hash, error)) return false;
  if (hash != binary.kernel_hash) {
    error = "code object " + binary.so_path + " changed since it was cached (hash " + hash + ", expected " +
            binary.kernel_hash + "); re-run the autotuner";
    return false;
  }
  hipModule_t m = nullptr;
  const hipError_t e = hipModuleLoad(&m, binary.so_path.c_str());
  if (e != hipSuccess) {
    error = "hipModuleLoad(" + binary.so_path + ") failed: " + hipGetErrorString(e);
    (void)hipGetLastError();
    return false;
  }
  if (module_) (void)hipModuleUnload(static_cast<hipModule_t>(module_));
  module_ = m;
  return true;
}

void *CodeObject::Function(std::string_view name, std::string &error) const {
  if (!module_) {
    error = "code object not loaded";
    return nullptr;
  }
  hipFunction_t f = nullptr;
  const hipError_t e = hipModuleGetFunction(&f, static_cast<hipModule_t>(module_), std::string(name).c_str());
  if (e != hipSuccess) {
    error = "kernel " + std::string(name) + " not found in code object: " + hipGetErrorString(e);
    (void)hipGetLastError();
    return nullptr;
  }
  return reinterpret_cast<void *>(f);
}

}  // namespace pk::runtime

namespace pk::autotune {

HipEventTimer::HipEventTimer() {
  hipEvent_t a = nullptr, b = nullptr;
  if (hipEventCreate(&a) == hipSuccess && hipEventCreate(&b) == hipSuccess) {
    start_ = a;
    stop_ = b;
  } else {
    if (a) (void)hipEventDestroy(a);
    (void)hipGetLastError();
  }
}

HipEventTimer::~HipEventTimer() {
  if (start_) (void)hipEventDestroy(static_cast<hipEvent_t>(start_));
  if (stop_) (void)hipEventDestroy(static_cast<hipEvent_t>(stop_));
}

void HipEventTimer::Start(void *s) {
  if (start_) (void)hipEventRecord(static_cast<hipEvent_t>(start_), static_cast<hipStream_t>(s));
}

void HipEventTimer::Stop(void *s) {
  if (stop_) (void)hipEventRecord(static_cast<hipEvent_t>(stop_), static_cast<hipStream_t>(s));
}

float HipEventTimer::ElapsedMs() {
  if (!ok()) return -1.0f;
  if (hipEventSynchronize(static_cast<hipEvent_t>(stop_)) != hipSuccess) return -1.0f;
  float ms = 0.0f;
  if (hipEventElapsedTime(&ms, static_cast<hipEvent_t>(start_), static_cast<hipEvent_t>(stop_)) != hipSuccess)
    return -1.0f;
  return ms;
}

}  // namespace pk::autotune
