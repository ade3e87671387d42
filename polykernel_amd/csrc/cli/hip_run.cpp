// hip_run.cpp -- pk_hip_run: run one op of the gfx950 library on .npy files.
//
// The command-line contract of the reference's hip_run driver
// (lib/Runtime/hip_run_main.cpp:17-27, 313-337), so its harnesses drive these
// kernels unchanged:
//   pk_hip_run rmsnorm IN OUT [--weight W] [--epsilon E]     (eps default 1e-5)
//   pk_hip_run gelu IN OUT
//   pk_hip_run matmul A B C
//   pk_hip_run softmax IN OUT [--axis A]                     (last axis only)
//   pk_hip_run fused_rmsnorm_matmul X W OUT [--epsilon E] [--weight G]
//   pk_hip_run fused_matmul_bias_gelu A B BIAS OUT
//   pk_hip_run neg                                           (invalid launch probe)
// plus the ops of this library the reference has only as golden compositions:
//   pk_hip_run fused_matmul_bias_residual A B BIAS R OUT
//   pk_hip_run fused_residual_rmsnorm X R OUT [--weight W] [--epsilon E]
//   pk_hip_run fused_softmax_mask LOGITS(<f4) MASK OUT
//   pk_hip_run quantize W WQ(|i1) SCALE(<f4)
//   pk_hip_run matmul_int8 A WQ SCALE C
//   pk_hip_run attention_prefill Q K V O [--scale S] [--causal 0|1]
//   pk_hip_run kv_cache_update CACHE NEW OUT
//   pk_hip_run fused_kv_append_attention Q KC VC KN VN O [--scale S] [--causal 0|1]
//              [--kc-out F] [--vc-out F]
// and two file utilities that need no GPU:
//   pk_hip_run info IN          (dtype and shape)
//   pk_hip_run roundtrip IN OUT (read, then write with this bridge's writer)
// bf16 files are '<V2' (raw bits), int8 '|i1', fp32 '<f4'.  Leading dims are
// flattened into rows (the reference's convention).  Exit status: 0 success,
// 1 error (reported on stderr; `neg` exits 1 when the invalid launch is
// caught), 2 usage error or an invalid launch that was accepted.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <map>
#include <string>
#include <vector>

#include "../../../include/polykernel_amd.h"
#include "npy.hpp"

namespace {

struct Failure : std::runtime_error {
  using std::runtime_error::runtime_error;
};

void Hip(hipError_t e, const char *what) {
  if (e != hipSuccess) throw Failure(std::string(what) + ": " + hipGetErrorString(e));
}

void Pk(int rc, const char *what) {
  if (rc != PK_OK) throw Failure(std::string(what) + " failed (status " + std::to_string(rc) + "): " + pk_last_error());
}

// A device copy of a host array (or an uninitialised device buffer).
struct Dev {
  void *p = nullptr;
  size_t bytes = 0;
  explicit Dev(size_t n) : bytes(n) {
    if (n) Hip(hipMalloc(&p, n), "hipMalloc");
  }
  explicit Dev(const pk::npy::Array &a) : Dev(a.data.size()) {
    if (bytes) Hip(hipMemcpy(p, a.data.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
  }
  ~Dev() {
    if (p) (void)hipFree(p);
  }
  Dev(const Dev &) = delete;
  Dev &operator=(const Dev &) = delete;
  template <typename T>
  T *as() const {
    return static_cast<T *>(p);
  }
};

void Save(const Dev &d, const std::string &descr, const std::vector<int64_t> &shape, const std::string &path) {
  std::vector<uint8_t> host(d.bytes);
  if (d.bytes) Hip(hipMemcpy(host.data(), d.p, d.bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  pk::npy::Write(path, descr, shape, host.data());
}

const std::vector<std::string> kBf16 = {"<V2", "<u2", "<i2"};

struct Args {
  std::vector<std::string> pos;
  std::map<std::string, std::string> opt;
  std::string Opt(const std::string &k, const std::string &def) const {
    const auto it = opt.find(k);
    return it == opt.end() ? def : it->second;
  }
};

int Rows(const pk::npy::Array &a) {
  if (a.shape.empty()) throw Failure("a 0-d array has no rows");
  return (int)(a.size() / a.shape.back());
}
int Cols(const pk::npy::Array &a) {
  if (a.shape.empty()) throw Failure("a 0-d array has no columns");
  return (int)a.shape.back();
}
std::vector<int64_t> MatmulOut(const std::vector<int64_t> &a, int64_t n) {
  std::vector<int64_t> s(a.begin(), a.end() - 1);
  s.push_back(n);
  return s;
}
void Need(bool ok, const std::string &msg) {
  if (!ok) throw Failure(msg);
}
void Sync() { Hip(hipDeviceSynchronize(), "hipDeviceSynchronize"); }

struct Op {
  int npos;
  const char *usage;
  std::vector<std::string> opts;
  std::function<int(const Args &)> run;
};

int RunNeg(const Args &) {
  int launch = 0, sync = 0;
  const int rc = pk_probe_invalid_launch(&launch, &sync);
  std::fprintf(stderr, "[polykernel-hip] neg: launch-config error = %s\n", hipGetErrorString((hipError_t)launch));
  std::fprintf(stderr, "[polykernel-hip] neg: sync error          = %s\n", hipGetErrorString((hipError_t)sync));
  if (rc != PK_OK) {
    std::fprintf(stderr, "[polykernel-hip] neg: FAIL - invalid launch produced NO error\n");
    return 2;
  }
  std::fprintf(stderr, "[polykernel-hip] neg: PASS - invalid launch CAUGHT + reported; no output written, no crash\n");
  return 1;
}

std::map<std::string, Op> Ops() {
  using pk::npy::Array;
  using pk::npy::Read;
  std::map<std::string, Op> ops;
  ops["info"] = {1, "info IN", {}, [](const Args &a) {
                   const Array x = Read(a.pos[0]);
                   std::printf("descr=%s shape=%s\n", x.descr.c_str(), pk::npy::detail::ShapeRepr(x.shape).c_str());
                   return 0;
                 }};
  ops["roundtrip"] = {2, "roundtrip IN OUT", {}, [](const Args &a) {
                        const Array x = Read(a.pos[0]);
                        pk::npy::Write(a.pos[1], x.descr, x.shape, x.data.data());
                        return 0;
                      }};
  ops["neg"] = {0, "neg", {}, RunNeg};
  ops["rmsnorm"] = {2, "rmsnorm IN OUT [--weight W] [--epsilon E]", {"--weight", "--epsilon"}, [](const Args &a) {
                      const Array x = Read(a.pos[0], kBf16);
                      const std::string wp = a.Opt("--weight", "");
                      Array w;
                      if (!wp.empty()) {
                        w = Read(wp, kBf16);
                        Need(w.size() == Cols(x), "rmsnorm: weight length != cols");
                      }
                      Dev dx(x), dw(w), dy(x.data.size());
                      Pk(launch_rmsnorm(dx.as<uint16_t>(), wp.empty() ? nullptr : dw.as<uint16_t>(), dy.as<uint16_t>(),
                                        Rows(x), Cols(x), std::stof(a.Opt("--epsilon", "1e-5")), nullptr),
                         "launch_rmsnorm");
                      Sync();
                      Save(dy, "<V2", x.shape, a.pos[1]);
                      return 0;
                    }};
  ops["gelu"] = {2, "gelu IN OUT", {}, [](const Args &a) {
                   const Array x = Read(a.pos[0], kBf16);
                   Dev dx(x), dy(x.data.size());
                   Pk(launch_gelu(dx.as<uint16_t>(), dy.as<uint16_t>(), (int)x.size(), nullptr), "launch_gelu");
                   Sync();
                   Save(dy, "<V2", x.shape, a.pos[1]);
                   return 0;
                 }};
  ops["matmul"] = {3, "matmul A B C", {}, [](const Args &a) {
                     const Array A = Read(a.pos[0], kBf16), B = Read(a.pos[1], kBf16);
                     Need(B.shape.size() == 2 && B.shape[0] == Cols(A), "matmul: contraction mismatch A.K != B.K");
                     const int M = Rows(A), K = Cols(A), N = (int)B.shape[1];
                     Dev da(A), db(B), dc((size_t)M * N * 2);
                     Pk(launch_matmul(da.as<uint16_t>(), db.as<uint16_t>(), dc.as<uint16_t>(), M, N, K, nullptr),
                        "launch_matmul");
                     Sync();
                     Save(dc, "<V2", MatmulOut(A.shape, N), a.pos[2]);
                     return 0;
                   }};
  ops["softmax"] = {2, "softmax IN OUT [--axis A]", {"--axis"}, [](const Args &a) {
                      const Array x = Read(a.pos[0], kBf16);
                      const int axis = std::stoi(a.Opt("--axis", "-1"));
                      Need(axis == -1 || axis == (int)x.shape.size() - 1, "softmax: only last-axis reduction (axis=-1)");
                      Dev dx(x), dy(x.data.size());
                      Pk(launch_softmax(dx.as<uint16_t>(), dy.as<uint16_t>(), Rows(x), Cols(x), nullptr), "launch_softmax");
                      Sync();
                      Save(dy, "<V2", x.shape, a.pos[1]);
                      return 0;
                    }};
  ops["fused_rmsnorm_matmul"] = {
      3, "fused_rmsnorm_matmul X W OUT [--epsilon E] [--weight G]", {"--epsilon", "--weight"}, [](const Args &a) {
        const Array x = Read(a.pos[0], kBf16), w = Read(a.pos[1], kBf16);
        Need(w.shape.size() == 2 && w.shape[0] == Cols(x), "fused_rmsnorm_matmul: K mismatch X.K != W.K");
        const int M = Rows(x), K = Cols(x), N = (int)w.shape[1];
        const std::string gp = a.Opt("--weight", "");
        Array g;
        if (!gp.empty()) {
          g = Read(gp, kBf16);
          Need(g.size() == K, "fused_rmsnorm_matmul: gamma length != K");
        }
        Dev dx(x), dw(w), dg(g), dy((size_t)M * N * 2);
        Pk(launch_fused_rmsnorm_matmul_gamma(dx.as<uint16_t>(), gp.empty() ? nullptr : dg.as<uint16_t>(),
                                             dw.as<uint16_t>(), dy.as<uint16_t>(), M, N, K,
                                             std::stof(a.Opt("--epsilon", "1e-5")), nullptr),
           "launch_fused_rmsnorm_matmul");
        Sync();
        Save(dy, "<V2", MatmulOut(x.shape, N), a.pos[2]);
        return 0;
      }};
  ops["fused_matmul_bias_gelu"] = {4, "fused_matmul_bias_gelu A B BIAS OUT", {}, [](const Args &a) {
                                     const Array A = Read(a.pos[0], kBf16), B = Read(a.pos[1], kBf16),
                                                 bias = Read(a.pos[2], kBf16);
                                     Need(B.shape.size() == 2 && B.shape[0] == Cols(A), "K mismatch");
                                     const int M = Rows(A), K = Cols(A), N = (int)B.shape[1];
                                     Need(bias.size() == N, "bias length != N");
                                     Dev da(A), db(B), dbias(bias), dc((size_t)M * N * 2);
                                     Pk(launch_fused_matmul_bias_gelu(da.as<uint16_t>(), db.as<uint16_t>(),
                                                                      dbias.as<uint16_t>(), dc.as<uint16_t>(), M, N, K,
                                                                      nullptr),
                                        "launch_fused_matmul_bias_gelu");
                                     Sync();
                                     Save(dc, "<V2", MatmulOut(A.shape, N), a.pos[3]);
                                     return 0;
                                   }};
  ops["fused_matmul_bias_residual"] = {
      5, "fused_matmul_bias_residual A B BIAS R OUT", {}, [](const Args &a) {
        const Array A = Read(a.pos[0], kBf16), B = Read(a.pos[1], kBf16), bias = Read(a.pos[2], kBf16),
                    R = Read(a.pos[3], kBf16);
        Need(B.shape.size() == 2 && B.shape[0] == Cols(A), "K mismatch");
        const int M = Rows(A), K = Cols(A), N = (int)B.shape[1];
        Need(bias.size() == N && R.size() == (int64_t)M * N, "bias / residual shape mismatch");
        Dev da(A), db(B), dbias(bias), dr(R), dc((size_t)M * N * 2);
        Pk(launch_fused_matmul_bias_residual(da.as<uint16_t>(), db.as<uint16_t>(), dbias.as<uint16_t>(),
                                             dr.as<uint16_t>(), dc.as<uint16_t>(), M, N, K, nullptr),
           "launch_fused_matmul_bias_residual");
        Sync();
        Save(dc, "<V2", MatmulOut(A.shape, N), a.pos[4]);
        return 0;
      }};
  ops["fused_residual_rmsnorm"] = {
      3, "fused_residual_rmsnorm X R OUT [--weight W] [--epsilon E]", {"--weight", "--epsilon"}, [](const Args &a) {
        const Array x = Read(a.pos[0], kBf16), r = Read(a.pos[1], kBf16);
        Need(r.size() == x.size(), "residual shape mismatch");
        const std::string wp = a.Opt("--weight", "");
        Array w;
        if (!wp.empty()) {
          w = Read(wp, kBf16);
          Need(w.size() == Cols(x), "weight length != cols");
        }
        Dev dx(x), dr(r), dw(w), dy(x.data.size());
        Pk(launch_fused_residual_rmsnorm(dx.as<uint16_t>(), dr.as<uint16_t>(), wp.empty() ? nullptr : dw.as<uint16_t>(),
                                         dy.as<uint16_t>(), Rows(x), Cols(x), std::stof(a.Opt("--epsilon", "1e-5")),
                                         nullptr),
           "launch_fused_residual_rmsnorm");
        Sync();
        Save(dy, "<V2", x.shape, a.pos[2]);
        return 0;
      }};
  ops["fused_softmax_mask"] = {3, "fused_softmax_mask LOGITS MASK OUT", {}, [](const Args &a) {
                                 const Array x = Read(a.pos[0], {"<f4"}), m = Read(a.pos[1], kBf16);
                                 Need(m.size() == x.size(), "mask shape mismatch");
                                 Dev dx(x), dm(m), dy((size_t)x.size() * 2);
                                 Pk(launch_fused_softmax_mask(dx.as<float>(), dm.as<uint16_t>(), dy.as<uint16_t>(),
                                                              Rows(x), Cols(x), nullptr),
                                    "launch_fused_softmax_mask");
                                 Sync();
                                 Save(dy, "<V2", x.shape, a.pos[2]);
                                 return 0;
                               }};
  ops["quantize"] = {3, "quantize W WQ SCALE", {}, [](const Args &a) {
                       const Array w = Read(a.pos[0], kBf16);
                       Need(w.shape.size() == 2, "quantize: W must be [K, N]");
                       const int K = (int)w.shape[0], N = (int)w.shape[1];
                       Dev dw(w), dq((size_t)K * N), ds((size_t)N * 4);
                       Pk(launch_quantize_int8_per_channel(dw.as<uint16_t>(), dq.as<int8_t>(), ds.as<float>(), K, N,
                                                           nullptr),
                          "launch_quantize_int8_per_channel");
                       Sync();
                       Save(dq, "|i1", w.shape, a.pos[1]);
                       Save(ds, "<f4", {N}, a.pos[2]);
                       return 0;
                     }};
  ops["matmul_int8"] = {4, "matmul_int8 A WQ SCALE C", {}, [](const Args &a) {
                          const Array A = Read(a.pos[0], kBf16), W = Read(a.pos[1], {"|i1"}),
                                      s = Read(a.pos[2], {"<f4"});
                          Need(W.shape.size() == 2 && W.shape[0] == Cols(A), "matmul_int8: K mismatch");
                          const int M = Rows(A), K = Cols(A), N = (int)W.shape[1];
                          Need(s.size() == N, "matmul_int8: scale length != N");
                          Dev da(A), dw(W), ds(s), dc((size_t)M * N * 2);
                          Pk(launch_matmul_int8(da.as<uint16_t>(), dw.as<int8_t>(), ds.as<float>(), dc.as<uint16_t>(),
                                                M, N, K, nullptr),
                             "launch_matmul_int8");
                          Sync();
                          Save(dc, "<V2", MatmulOut(A.shape, N), a.pos[3]);
                          return 0;
                        }};
  ops["attention_prefill"] = {
      4, "attention_prefill Q K V O [--scale S] [--causal 0|1]", {"--scale", "--causal"}, [](const Args &a) {
        const Array q = Read(a.pos[0], kBf16), k = Read(a.pos[1], kBf16), v = Read(a.pos[2], kBf16);
        Need(q.shape.size() == 4 && k.shape.size() == 4 && k.shape == v.shape, "attention: Q, K, V must be [B,H,S,D]");
        const int B = (int)q.shape[0], H = (int)q.shape[1], Sq = (int)q.shape[2], D = (int)q.shape[3];
        const int Skv = (int)k.shape[2];
        Need(k.shape[0] == B && k.shape[1] == H && k.shape[3] == D, "attention: K/V batch, heads or D mismatch");
        const float scale = std::stof(a.Opt("--scale", std::to_string(1.0f / std::sqrt((float)D))));
        Dev dq(q), dk(k), dv(v), dout(q.data.size());
        Pk(launch_attention_prefill(dq.as<uint16_t>(), dk.as<uint16_t>(), dv.as<uint16_t>(), dout.as<uint16_t>(), B, H,
                                    Sq, Skv, D, scale, std::stoi(a.Opt("--causal", "1")), nullptr),
           "launch_attention_prefill");
        Sync();
        Save(dout, "<V2", q.shape, a.pos[3]);
        return 0;
      }};
  ops["kv_cache_update"] = {3, "kv_cache_update CACHE NEW OUT", {}, [](const Args &a) {
                              const Array c = Read(a.pos[0], kBf16), n = Read(a.pos[1], kBf16);
                              Need(c.shape.size() == 4 && n.shape.size() == 4 && c.shape[0] == n.shape[0] &&
                                       c.shape[1] == n.shape[1] && c.shape[3] == n.shape[3],
                                   "kv_cache_update: [B,H,S,D] shapes mismatch");
                              std::vector<int64_t> os = c.shape;
                              os[2] += n.shape[2];
                              Dev dc(c), dn(n), dout((size_t)os[0] * os[1] * os[2] * os[3] * 2);
                              Pk(launch_kv_cache_update(dc.as<uint16_t>(), dn.as<uint16_t>(), dout.as<uint16_t>(),
                                                        (int)c.shape[0], (int)c.shape[1], (int)c.shape[2],
                                                        (int)n.shape[2], (int)c.shape[3], nullptr),
                                 "launch_kv_cache_update");
                              Sync();
                              Save(dout, "<V2", os, a.pos[2]);
                              return 0;
                            }};
  ops["fused_kv_append_attention"] = {
      6, "fused_kv_append_attention Q KC VC KN VN O [--scale S] [--causal 0|1] [--kc-out F] [--vc-out F]",
      {"--scale", "--causal", "--kc-out", "--vc-out"}, [](const Args &a) {
        // KC/VC hold the valid cache rows [B,H,S_cache,D]; the device copies get
        // room for S_cache + S_q rows and the append happens in place there.
        const Array q = Read(a.pos[0], kBf16), kc = Read(a.pos[1], kBf16), vc = Read(a.pos[2], kBf16),
                    kn = Read(a.pos[3], kBf16), vn = Read(a.pos[4], kBf16);
        Need(q.shape.size() == 4 && kc.shape.size() == 4 && kc.shape == vc.shape && kn.shape == q.shape &&
                 vn.shape == q.shape,
             "fused_kv_append_attention: Q/KN/VN [B,H,S_q,D], KC/VC [B,H,S_cache,D]");
        const int B = (int)q.shape[0], H = (int)q.shape[1], Sq = (int)q.shape[2], D = (int)q.shape[3];
        const int Sc = (int)kc.shape[2], cap = Sc + Sq;
        const size_t row = (size_t)D * 2, bh = (size_t)B * H;
        Dev dkc(bh * cap * row), dvc(bh * cap * row), dq(q), dkn(kn), dvn(vn), dout(q.data.size());
        for (size_t i = 0; i < bh; ++i) {  // cache rows into the capacity layout
          Hip(hipMemcpy(dkc.as<uint8_t>() + i * cap * row, kc.data.data() + i * Sc * row, Sc * row, hipMemcpyHostToDevice),
              "hipMemcpy");
          Hip(hipMemcpy(dvc.as<uint8_t>() + i * cap * row, vc.data.data() + i * Sc * row, Sc * row, hipMemcpyHostToDevice),
              "hipMemcpy");
        }
        const float scale = std::stof(a.Opt("--scale", std::to_string(1.0f / std::sqrt((float)D))));
        Pk(launch_fused_kv_append_attention(dq.as<uint16_t>(), dkc.as<uint16_t>(), dvc.as<uint16_t>(),
                                            dkn.as<uint16_t>(), dvn.as<uint16_t>(), dout.as<uint16_t>(), B, H, Sq, Sc,
                                            D, cap, scale, std::stoi(a.Opt("--causal", "1")), nullptr),
           "launch_fused_kv_append_attention");
        Sync();
        Save(dout, "<V2", q.shape, a.pos[5]);
        const std::vector<int64_t> cs = {B, H, cap, D};
        if (!a.Opt("--kc-out", "").empty()) Save(dkc, "<V2", cs, a.Opt("--kc-out", ""));
        if (!a.Opt("--vc-out", "").empty()) Save(dvc, "<V2", cs, a.Opt("--vc-out", ""));
        return 0;
      }};
  return ops;
}

int Usage(const std::map<std::string, Op> &ops, const std::string &msg) {
  std::fprintf(stderr, "usage: pk_hip_run <op> ...   (%s)\n", msg.c_str());
  for (const auto &[name, op] : ops) std::fprintf(stderr, "  pk_hip_run %s\n", op.usage);
  return 2;
}

}  // namespace

int main(int argc, char **argv) {
  const std::map<std::string, Op> ops = Ops();
  if (argc < 2) return Usage(ops, "no op");
  const auto it = ops.find(argv[1]);
  if (it == ops.end()) return Usage(ops, std::string("unknown op ") + argv[1]);
  const Op &op = it->second;
  Args args;
  for (int i = 2; i < argc; ++i) {
    const std::string s = argv[i];
    if (s.rfind("--", 0) == 0) {
      if (std::find(op.opts.begin(), op.opts.end(), s) == op.opts.end() || i + 1 >= argc)
        return Usage(ops, "bad option " + s + " for " + argv[1]);
      args.opt[s] = argv[++i];
    } else {
      args.pos.push_back(s);
    }
  }
  if ((int)args.pos.size() != op.npos) return Usage(ops, op.usage);
  try {
    return op.run(args);
  } catch (const std::exception &e) {
    std::fprintf(stderr, "[polykernel-hip] error: %s\n", e.what());
    return 1;
  }
}
