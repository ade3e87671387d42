// core.hip -- library state behind the C-ABI: error messages, per-device GELU
// table, library-owned workspace, device/arch detection, synthetic inputs.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <tuple>
#include <vector>

#include "pk_common.hpp"

namespace pk {

namespace {
thread_local char g_err[512] = "";
constexpr int kMaxDevices = 64;

std::mutex g_mu;
bool g_table_ready[kMaxDevices] = {};
const uint16_t *g_table_ptr[kMaxDevices] = {};

// One workspace slot per (device, stream); buffers a slot outgrew stay
// allocated beside it (`retired`) until pk_release_workspace frees the slot
// (or the process ends).  hipStreamPerThread names a different stream on
// every host thread, so its slots are keyed by thread as well.  Leases hold a
// reference, so a slot released while another thread waits for it stays
// valid; that thread then sees `released` and takes the new slot.
struct WsSlot {
  std::mutex mu;
  void *ptr = nullptr;
  size_t bytes = 0;
  std::vector<void *> retired;
  bool released = false;
};
using WsKey = std::tuple<int, uintptr_t, size_t>;
std::map<WsKey, std::shared_ptr<WsSlot>> g_ws_slots;  // guarded by g_mu

WsKey ws_key(int dev, void *st) {
  const size_t thread_tag =
      st == (void *)hipStreamPerThread ? std::hash<std::thread::id>{}(std::this_thread::get_id()) : 0;
  return WsKey{dev, reinterpret_cast<uintptr_t>(st), thread_tag};
}
}  // namespace

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

int hip_fail(hipError_t e, const char *what) {
  set_error("%s failed: %s", what, hipGetErrorString(e));
  return e == hipErrorNoDevice ? PK_ERR_NO_DEVICE : PK_ERR_HIP;
}

// The compact GELU table (pk_common.hpp, gelu_bits): entry i is the bf16 GELU
// of gelu_table_code(i) (or that slot's sentinel), evaluated as
// kernels/cpu/cpu_reference.cpp:46-55 does:
// e = (float)erf((double)(x * 0.70710678f)); y = bf16((0.5f * x) * (1.0f + e)).
__device__ uint16_t g_gelu_table_storage[GELU_TABLE_SIZE];

__global__ void gelu_table_init_kernel(uint16_t *tab) {
#pragma clang fp contract(off)
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= GELU_TABLE_SIZE) return;
  bool sentinel;
  const uint32_t code = gelu_table_code(i, &sentinel);
  if (sentinel) {
    tab[i] = (uint16_t)code;
    return;
  }
  const float kInvSqrt2 = 0.70710678118654752440f;
  const float x = bf2f(code);
  const float e = (float)erf((double)(x * kInvSqrt2));
  const float y = (0.5f * x) * (1.0f + e);
  tab[i] = (uint16_t)f2bf(y);
}

// Exhaustive device self-check: f2bf (hardware conversion) against the
// reference formula over all 2^32 fp32 bit patterns.
__global__ void bf16_selfcheck_kernel(unsigned long long *bad) {
  const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  unsigned long long n = 0;
  for (uint32_t j = 0; j < 1024; ++j) {
    const uint32_t u = (uint32_t)(tid * 1024u + j);
    n += f2bf(__uint_as_float(u)) != f2bf_formula(__uint_as_float(u));
  }
  if (n) atomicAdd(bad, n);
}

// Self-check of the paired GELU: for every low code (all 65536) and four
// high-code patterns, gelu_pair_common (where gelu_pair_special finds neither
// code outside its domain) and the dispatch the GEMM epilogue uses must equal
// gelu_bits of each code, and the epilogue's accumulated vote (GeluVote) must
// flag exactly the pairs gelu_pair_special flags.
__global__ void gelu_pair_selfcheck_kernel(const uint16_t *tab, unsigned long long *bad) {
  const uint32_t lo = blockIdx.x * blockDim.x + threadIdx.x;
  if (lo >= 65536u) return;
  unsigned long long n = 0;
  const uint32_t his[4] = {lo, lo ^ 0x8000u, (lo * 40503u + 7u) & 0xFFFFu, 0xFFFFu - lo};
  for (int k = 0; k < 4; ++k) {
    const uint32_t w = lo | (his[k] << 16);
    const uint32_t want = gelu_pair_exact(w, tab);
    if (!gelu_pair_special(w)) n += gelu_pair_common(w, tab) != want;
    const uint32_t got = gelu_pair_special(w) ? gelu_pair_exact(w, tab) : gelu_pair_common(w, tab);
    n += got != want;
    // the accumulated vote of the GEMM epilogue agrees with gelu_pair_special
    GeluVote v = gelu_vote_init();
    gelu_vote_add(v, w & 0x7FFF7FFFu);
    n += gelu_vote_special(v) != (gelu_pair_special(w) != 0u);
  }
  if (n) atomicAdd(bad, n);
}

int gelu_table(const uint16_t **table) {
  int dev = 0;
  PK_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("device ordinal %d out of range", dev);
    return PK_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_table_ready[dev]) {
    void *p = nullptr;
    PK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(g_gelu_table_storage)));
    uint16_t *tab = static_cast<uint16_t *>(p);
    gelu_table_init_kernel<<<(GELU_TABLE_SIZE + 255) / 256, 256, 0, nullptr>>>(tab);
    PK_LAUNCH_CHECK("gelu_table_init_kernel");
    // One-time set-up: make the table visible to every stream before use.
    PK_HIP(hipDeviceSynchronize());
    g_table_ptr[dev] = tab;
    g_table_ready[dev] = true;
  }
  *table = g_table_ptr[dev];
  return PK_OK;
}

int library_workspace(size_t bytes, void *st, WorkspaceLease &lease) {
  int dev = 0;
  PK_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("device ordinal %d out of range", dev);
    return PK_ERR_UNSUPPORTED;
  }
  const WsKey key = ws_key(dev, st);
  std::shared_ptr<WsSlot> slot;
  std::unique_lock<std::mutex> lk;
  for (;;) {
    {
      std::lock_guard<std::mutex> g(g_mu);
      std::shared_ptr<WsSlot> &s = g_ws_slots[key];
      if (!s) s = std::make_shared<WsSlot>();
      slot = s;
    }
    lk = std::unique_lock<std::mutex>(slot->mu);
    if (!slot->released) break;
    lk.unlock();  // released between the lookup and the lock: take the slot that replaced it
  }
  if (slot->bytes < bytes) {
    size_t want = size_t(1) << 20;
    while (want < bytes) want <<= 1;
    void *p = nullptr;
    PK_HIP(hipMalloc(&p, want));
    if (slot->ptr) slot->retired.push_back(slot->ptr);
    slot->ptr = p;
    slot->bytes = want;
  }
  lease.ptr = slot->ptr;
  lease.keep = slot;
  lease.lock = std::move(lk);
  return PK_OK;
}

int release_workspace(void *st) {
  int dev = 0;
  PK_HIP(hipGetDevice(&dev));
  std::shared_ptr<WsSlot> slot;
  {
    std::lock_guard<std::mutex> g(g_mu);
    auto it = g_ws_slots.find(ws_key(dev, st));
    if (it == g_ws_slots.end()) return PK_OK;
    slot = it->second;
    g_ws_slots.erase(it);
  }
  // wait for a lease holder to finish enqueuing, then for the stream's
  // queued kernels (the last readers of the buffers) before freeing them
  std::lock_guard<std::mutex> lk(slot->mu);
  slot->released = true;
  PK_HIP(hipStreamSynchronize(static_cast<hipStream_t>(st)));
  for (void *p : slot->retired) PK_HIP(hipFree(p));
  slot->retired.clear();
  if (slot->ptr) PK_HIP(hipFree(slot->ptr));
  slot->ptr = nullptr;
  slot->bytes = 0;
  return PK_OK;
}

// ---- synthetic generator ---------------------------------------------------
namespace {
inline uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint64_t stream_id) {
  return splitmix64(seed ^ (stream_id * 0xD1B54A32D192ED03ull));
}

// Standard normal draw i of a (seed, stream) pair: Box-Muller in double on two
// 53-bit uniforms; u1 in (0,1], u2 in [0,1).
inline double normal_at(uint64_t key, int64_t i) {
  const uint64_t a = splitmix64(key + 2ull * (uint64_t)i);
  const uint64_t b = splitmix64(key + 2ull * (uint64_t)i + 1ull);
  const double u1 = (double)((a >> 11) + 1ull) * 0x1.0p-53;
  const double u2 = (double)(b >> 11) * 0x1.0p-53;
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586476925 * u2);
}

inline uint16_t host_f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0u)
    return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <typename F>
void parallel_for(int64_t n, F &&f) {
  unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  int64_t nt = std::min<int64_t>(hw, std::max<int64_t>(1, n / 65536));
  if (nt <= 1) {
    f(0, n);
    return;
  }
  std::vector<std::thread> th;
  int64_t chunk = (n + nt - 1) / nt;
  for (int64_t t = 0; t < nt; ++t) {
    int64_t lo = t * chunk, hi = std::min(n, lo + chunk);
    if (lo >= hi) break;
    th.emplace_back([=, &f] { f(lo, hi); });
  }
  for (auto &x : th) x.join();
}
}  // namespace

// One in-bounds store: the kernel of the invalid-launch probe.
__global__ void probe_store_kernel(uint16_t *out) {
  if (blockIdx.x == 0 && threadIdx.x == 0) out[0] = 0x3F80u;
}

// The launch-floor probe: no memory access; the dynamic LDS is reserved by
// the launch (the never-taken store keeps the declaration live).
__global__ void probe_empty_kernel(int never) {
  extern __shared__ uint32_t probe_lds[];
  if (never == 1) probe_lds[threadIdx.x] = 0u;
}

}  // namespace pk

using namespace pk;

extern "C" {

// Launch probe_store_kernel with 2048 threads per workgroup -- twice the
// gfx950 limit -- and report what HIP says (lib/Runtime/hip_run_main.cpp:
// 278-309 of the reference).  The runtime rejects the configuration before
// dispatch; the kernel itself only ever writes out[0] of an 8-byte buffer.
int pk_probe_invalid_launch(int *launch_status, int *sync_status) {
  PK_CHECK_ARG(launch_status && sync_status, "pk_probe_invalid_launch: null argument");
  uint16_t *d = nullptr;
  PK_HIP(hipMalloc(&d, 8));
  probe_store_kernel<<<1, 2048, 0, nullptr>>>(d);
  const hipError_t le = hipGetLastError();
  const hipError_t se = hipDeviceSynchronize();
  (void)hipFree(d);
  *launch_status = (int)le;
  *sync_status = (int)se;
  (void)hipGetLastError();
  if (le == hipSuccess && se == hipSuccess) {
    set_error("pk_probe_invalid_launch: a 2048-thread workgroup was accepted");
    return PK_ERR_LAUNCH;
  }
  set_error("invalid launch caught: launch %s, sync %s", hipGetErrorString(le), hipGetErrorString(se));
  return PK_OK;
}

// An empty kernel at a given grid, workgroup size and dynamic LDS: the
// fixed cost of a launch of that geometry (dispatch, LDS allocation,
// workgroup start and retirement), timed beside latency-bound kernels.
int pk_probe_empty_launch(int blocks, int threads, int lds_bytes, void *stream) {
  PK_CHECK_ARG(blocks > 0 && threads > 0 && threads <= 1024 && lds_bytes >= 0 && lds_bytes <= 160 * 1024,
               "pk_probe_empty_launch: blocks %d, threads %d (1..1024), lds %d bytes (0..163840)", blocks,
               threads, lds_bytes);
  probe_empty_kernel<<<blocks, threads, (size_t)lds_bytes, (hipStream_t)stream>>>(0);
  PK_LAUNCH_CHECK("pk_probe_empty_launch");
  return PK_OK;
}

const char *pk_version(void) { return "polykernel_amd 0.1.0 gfx950"; }

const char *pk_last_error(void) { return g_err; }

int pk_gelu_table(const uint16_t **table) {
  if (!table) {
    set_error("pk_gelu_table: null argument");
    return PK_ERR_INVALID_ARG;
  }
  return gelu_table(table);
}

int pk_library_workspace(size_t bytes, void *stream, void **ptr) {
  if (!ptr) {
    set_error("pk_library_workspace: null argument");
    return PK_ERR_INVALID_ARG;
  }
  WorkspaceLease lease;
  int rc = library_workspace(bytes, stream, lease);
  if (rc == PK_OK) *ptr = lease.ptr;
  return rc;
}

int pk_release_workspace(void *stream) { return release_workspace(stream); }

int pk_init(void) {
  const uint16_t *t = nullptr;
  int rc = gelu_table(&t);
  if (rc) return rc;
  return int8_scratch_setup(nullptr);
}

int pk_check_bf16_conversion(unsigned long long *mismatches) {
  if (!mismatches) {
    set_error("pk_check_bf16_conversion: null argument");
    return PK_ERR_INVALID_ARG;
  }
  unsigned long long *d = nullptr;
  PK_HIP(hipMalloc(&d, sizeof(unsigned long long)));
  hipError_t e = hipMemset(d, 0, sizeof(unsigned long long));
  if (e == hipSuccess) {
    bf16_selfcheck_kernel<<<(1u << 22) / 256, 256>>>(d);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpy(mismatches, d, sizeof(unsigned long long), hipMemcpyDeviceToHost);
  hipFree(d);
  if (e != hipSuccess) return hip_fail(e, "pk_check_bf16_conversion");
  return PK_OK;
}

// Runs gelu_pair_selfcheck_kernel; the mismatch count goes to *mismatches.
int pk_check_gelu_pairs(unsigned long long *mismatches) {
  PK_CHECK_ARG(mismatches, "pk_check_gelu_pairs: null argument");
  const uint16_t *tab = nullptr;
  int rc = gelu_table(&tab);
  if (rc) return rc;
  unsigned long long *d = nullptr;
  PK_HIP(hipMalloc(&d, sizeof(unsigned long long)));
  hipError_t e = hipMemset(d, 0, sizeof(unsigned long long));
  if (e == hipSuccess) {
    gelu_pair_selfcheck_kernel<<<65536 / 256, 256>>>(tab, d);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpy(mismatches, d, sizeof(unsigned long long), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return hip_fail(e, "pk_check_gelu_pairs");
  return PK_OK;
}

// The bare arch token of a gcnArchName: from the first "gfx", when a digit
// follows it, through the run of lower-case letters and digits after it
// ("gfx950:sramecc+:xnack-" -> "gfx950"); "" otherwise
// (lib/Runtime/DeviceDetect.cpp:28-50 of the reference).
int pk_parse_gcn_arch_name(const char *name, char *buf, int buf_len) {
  if (!name || !buf || buf_len <= 0) {
    set_error("pk_parse_gcn_arch_name: null argument");
    return PK_ERR_INVALID_ARG;
  }
  buf[0] = '\0';
  const char *p = std::strstr(name, "gfx");
  if (!p || p[3] < '0' || p[3] > '9') return PK_OK;
  int n = 3;
  while ((p[n] >= '0' && p[n] <= '9') || (p[n] >= 'a' && p[n] <= 'z')) ++n;
  if (n + 1 > buf_len) {
    set_error("pk_parse_gcn_arch_name: buffer too small");
    return PK_ERR_INVALID_ARG;
  }
  std::memcpy(buf, p, n);
  buf[n] = '\0';
  return PK_OK;
}

// ---- configurations ---------------------------------------------------------

namespace {
enum OpFamily { OF_UNKNOWN, OF_GEMM, OF_INT8, OF_RMSNORM_MATMUL, OF_RMSNORM, OF_SOFTMAX, OF_ATTENTION };

OpFamily op_family(const char *op) {
  static const struct {
    const char *name;
    OpFamily family;
  } kOps[] = {{"matmul", OF_GEMM},
              {"fused_matmul_bias_gelu", OF_GEMM},
              {"fused_matmul_bias_residual", OF_GEMM},
              {"matmul_int8", OF_INT8},
              {"matmul_int8_gelu", OF_INT8},
              {"matmul_int8_residual", OF_INT8},
              {"fused_rmsnorm_matmul", OF_RMSNORM_MATMUL},
              {"fused_residual_rmsnorm", OF_RMSNORM},
              {"fused_softmax_mask", OF_SOFTMAX},
              {"fused_kv_append_attention", OF_ATTENTION}};
  if (!op) return OF_UNKNOWN;
  for (const auto &o : kOps)
    if (std::strcmp(op, o.name) == 0) return o.family;
  return OF_UNKNOWN;
}

bool dims_ok(long long M, long long N, long long K) {
  return M >= 0 && N >= 0 && K >= 0 && M <= INT32_MAX && N <= INT32_MAX && K <= INT32_MAX;
}

// One fixed configuration (or none) as a list.
int single(bool ok, const pk_config &c, pk_config *out, int cap) {
  if (!ok) return 0;
  if (out && cap > 0) out[0] = c;
  return 1;
}
}  // namespace

int pk_op_configs(const char *op, long long M, long long N, long long K, pk_config *out, int cap) {
  const OpFamily f = op_family(op);
  PK_CHECK_ARG(f != OF_UNKNOWN, "pk_op_configs: unknown op '%s'", op ? op : "(null)");
  PK_CHECK_ARG(cap >= 0 && (out || cap == 0), "pk_op_configs: invalid output buffer");
  if (!dims_ok(M, N, K)) return 0;
  const int m = (int)M, n = (int)N, k = (int)K;
  pk_config c{};
  switch (f) {
    case OF_GEMM: return gemm_configs(m, n, k, out, cap);
    case OF_INT8: return int8_configs(m, n, k, out, cap);
    case OF_RMSNORM_MATMUL: return single(rmsnorm_matmul_config(m, n, k, &c), c, out, cap);
    case OF_RMSNORM: return k == 0 ? rmsnorm_configs(m, n, out, cap) : 0;
    case OF_SOFTMAX: return k == 0 ? softmax_configs(m, n, out, cap) : 0;
    case OF_ATTENTION: return n >= m ? attention_configs(m, n, k, out, cap) : 0;
    default: return 0;
  }
}

int pk_op_default_config(const char *op, long long M, long long N, long long K, pk_config *out) {
  const OpFamily f = op_family(op);
  PK_CHECK_ARG(f != OF_UNKNOWN, "pk_op_default_config: unknown op '%s'", op ? op : "(null)");
  PK_CHECK_ARG(out != nullptr, "pk_op_default_config: null output");
  bool ok = false;
  if (dims_ok(M, N, K)) {
    const int m = (int)M, n = (int)N, k = (int)K;
    switch (f) {
      case OF_GEMM: ok = gemm_default(m, n, k, out); break;
      case OF_INT8: ok = int8_default(m, n, k, out); break;
      case OF_RMSNORM_MATMUL: ok = rmsnorm_matmul_config(m, n, k, out); break;
      case OF_RMSNORM: ok = k == 0 && rmsnorm_config(m, n, out); break;
      case OF_SOFTMAX: ok = k == 0 && softmax_config(m, n, out); break;
      case OF_ATTENTION: ok = n >= m && attention_config(m, n, k, out); break;
      default: break;
    }
  }
  if (!ok) {
    set_error("pk_op_default_config: %s has no configuration for M=%lld N=%lld K=%lld", op, M, N, K);
    return PK_ERR_UNSUPPORTED;
  }
  return PK_OK;
}

int pk_device_arch(int ordinal, char *buf, int buf_len) {
  hipDeviceProp_t p;
  hipError_t e = hipGetDeviceProperties(&p, ordinal);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  return pk_parse_gcn_arch_name(p.gcnArchName, buf, buf_len);
}

void pk_synth_normal_bf16(uint64_t seed, uint64_t stream_id, double mean, double std_dev,
                          uint16_t *out, int64_t n) {
  const uint64_t key = stream_key(seed, stream_id);
  parallel_for(n, [&](int64_t lo, int64_t hi) {
    for (int64_t i = lo; i < hi; ++i)
      out[i] = host_f2bf((float)(mean + std_dev * normal_at(key, i)));
  });
}

void pk_synth_normal_f32(uint64_t seed, uint64_t stream_id, double mean, double std_dev,
                         float *out, int64_t n) {
  const uint64_t key = stream_key(seed, stream_id);
  parallel_for(n, [&](int64_t lo, int64_t hi) {
    for (int64_t i = lo; i < hi; ++i) out[i] = (float)(mean + std_dev * normal_at(key, i));
  });
}

void pk_synth_mask_bf16(uint64_t seed, uint64_t stream_id, double p, uint16_t *out, int64_t n) {
  const uint64_t key = stream_key(seed, stream_id);
  parallel_for(n, [&](int64_t lo, int64_t hi) {
    for (int64_t i = lo; i < hi; ++i) {
      const double u = (double)(splitmix64(key + (uint64_t)i) >> 11) * 0x1.0p-53;
      out[i] = (u < p) ? (uint16_t)0xFF80u : (uint16_t)0x0000u;
    }
  });
}

}  // extern "C"
