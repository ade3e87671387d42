// parser_fuzz.cpp -- mutation fuzzing of the runtime's text parsers, built by
// tests/test_host_asan.py with the host sources of the runtime under
// AddressSanitizer and UndefinedBehaviorSanitizer (no GPU needed).
//
//   parser_fuzz TUNING_JSON CASES SEED SCRATCH_DIR
//
// Each case applies 1-8 random edits (delete, insert, overwrite with a
// JSON-significant byte, truncate) to the committed tuning cache and feeds the
// result to autotune::ParseTuningCache and runtime::KernelCache::
// LoadTuningCache; an accepted document must serialize and parse again.  The
// same edits are applied to a small .npy file read back by the CLI's reader
// (csrc/cli/npy.hpp), which must return an array or throw.  The sanitizers
// abort on any out-of-bounds access, use after free or undefined behaviour;
// the exit status is 0 when every case ran.
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <random>
#include <sstream>
#include <string>

#include "polykernel_amd_runtime.hpp"
#include "../../polykernel_amd/csrc/cli/npy.hpp"

int main(int argc, char **argv) {
  if (argc != 5) {
    std::fprintf(stderr, "usage: parser_fuzz TUNING_JSON CASES SEED SCRATCH_DIR\n");
    return 2;
  }
  std::ifstream in(argv[1], std::ios::binary);
  std::stringstream ss;
  ss << in.rdbuf();
  const std::string base = ss.str();
  if (base.empty()) {
    std::fprintf(stderr, "empty input %s\n", argv[1]);
    return 2;
  }
  const long cases = std::atol(argv[2]);
  std::mt19937_64 rng(std::strtoull(argv[3], nullptr, 10));
  static const char kSig[] = "{}[]\",:0123456789.-+eE truefalsn\\u\xff\xc3";
  auto mutate = [&](std::string s) {
    const int edits = 1 + static_cast<int>(rng() % 8);
    for (int e = 0; e < edits; ++e) {
      const size_t pos = rng() % (s.size() + 1);
      switch (rng() % 4) {
        case 0:
          if (!s.empty()) s.erase(std::min(pos, s.size() - 1), 1);
          break;
        case 1:
          s.insert(pos, 1, static_cast<char>(rng() % 256));
          break;
        case 2:
          if (!s.empty()) s[std::min(pos, s.size() - 1)] = kSig[rng() % (sizeof(kSig) - 1)];
          break;
        default:
          s.resize(pos);
      }
    }
    return s;
  };
  long accepted = 0, refused = 0;
  for (long c = 0; c < cases; ++c) {
    const std::string s = mutate(base);
    const pk::autotune::TuningCacheParseResult r = pk::autotune::ParseTuningCache(s);
    pk::runtime::KernelCache cache;
    std::string err;
    const bool loaded = cache.LoadTuningCache(s, err);
    if (r.ok()) {
      ++accepted;
      const pk::autotune::TuningCacheParseResult again =
          pk::autotune::ParseTuningCache(pk::autotune::SerializeTuningCache(*r.cache));
      if (!again.ok()) {
        std::fprintf(stderr, "case %ld: an accepted document does not survive a round trip\n", c);
        return 1;
      }
    } else {
      ++refused;
    }
    if (!loaded && err.empty()) {
      std::fprintf(stderr, "case %ld: refused without a message\n", c);
      return 1;
    }
  }
  // .npy: a valid [3, 4] fp32 file written by the CLI's own writer, then mutated
  const std::string npy_path = std::string(argv[4]) + "/fuzz.npy";
  const float vals[12] = {0.f, 1.f, 2.f, 3.f, 4.f, 5.f, 6.f, 7.f, 8.f, 9.f, 10.f, 11.f};
  pk::npy::Write(npy_path, "<f4", {3, 4}, vals);
  std::string npy;
  {
    std::ifstream f(npy_path, std::ios::binary);
    std::stringstream b;
    b << f.rdbuf();
    npy = b.str();
  }
  long npy_read = 0, npy_refused = 0;
  for (long c = 0; c < cases / 4; ++c) {
    const std::string m = mutate(npy);
    {
      std::ofstream f(npy_path, std::ios::binary | std::ios::trunc);
      f.write(m.data(), (std::streamsize)m.size());
    }
    try {
      const pk::npy::Array a = pk::npy::Read(npy_path);
      if (a.data.size() != (size_t)a.size() * (size_t)pk::npy::ItemSize(a.descr)) {
        std::fprintf(stderr, "npy case %ld: payload size does not match the shape\n", c);
        return 1;
      }
      ++npy_read;
    } catch (const std::exception &) {
      ++npy_refused;
    }
  }
  std::printf("cases %ld accepted %ld refused %ld npy_read %ld npy_refused %ld\n", cases, accepted, refused,
              npy_read, npy_refused);
  return 0;
}
