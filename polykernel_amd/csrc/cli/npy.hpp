// npy.hpp -- the .npy file bridge: bf16 as '<V2' (raw 16-bit patterns), int8
// as '|i1', fp32 as '<f4' (little-endian hosts).
//
// File format: NumPy format 1.0/2.0 (magic "\x93NUMPY", version, header
// length, a Python-literal dict with 'descr', 'fortran_order', 'shape').
// The writer produces the bytes the reference's writer produces
// (kernels/cpu/npy_io.cpp:127-171): version 1.0, the dict
// "{'descr': '<V2', 'fortran_order': False, 'shape': (2, 3), }" padded with
// spaces and a newline to a multiple of 64 bytes, so files are interchangeable
// with its harnesses; the reader takes what NumPy and that writer produce and
// refuses Fortran order and other dtypes.
#pragma once

#include <cstdint>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace pk::npy {

struct Array {
  std::string descr;           // "<V2" | "|i1" | "<f4"
  std::vector<int64_t> shape;  // C order
  std::vector<uint8_t> data;   // raw payload
  int64_t size() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
};

class Error : public std::runtime_error {
 public:
  using std::runtime_error::runtime_error;
};

inline int ItemSize(const std::string &descr) {
  if (descr == "<V2" || descr == "|V2" || descr == "<u2" || descr == "<i2") return 2;
  if (descr == "|i1" || descr == "|u1") return 1;
  if (descr == "<f4") return 4;
  return 0;
}

namespace detail {

// The quoted value following `key` ("'descr'") in the header dict.
inline std::string QuotedAfter(const std::string &h, const std::string &key) {
  const size_t k = h.find(key);
  if (k == std::string::npos) throw Error("npy header has no " + key);
  const size_t colon = h.find(':', k + key.size());
  if (colon == std::string::npos) throw Error("npy header: no value for " + key);
  size_t open = colon + 1;
  while (open < h.size() && h[open] == ' ') ++open;
  if (open >= h.size() || (h[open] != '\'' && h[open] != '"')) throw Error("npy header: " + key + " is not a string");
  const size_t close = h.find(h[open], open + 1);
  if (close == std::string::npos) throw Error("npy header: unterminated " + key);
  return h.substr(open + 1, close - open - 1);
}

inline std::vector<int64_t> Shape(const std::string &h) {
  const size_t k = h.find("'shape'");
  if (k == std::string::npos) throw Error("npy header has no 'shape'");
  const size_t open = h.find('(', k), close = h.find(')', open);
  if (open == std::string::npos || close == std::string::npos) throw Error("npy header: malformed 'shape'");
  std::vector<int64_t> shape;
  size_t i = open + 1;
  while (i < close) {
    while (i < close && (h[i] == ' ' || h[i] == ',')) ++i;
    if (i >= close) break;
    const size_t start = i;
    while (i < close && h[i] >= '0' && h[i] <= '9') ++i;
    if (i == start) throw Error("npy header: non-integer dimension in 'shape'");
    if (i - start > 15) throw Error("npy header: dimension " + h.substr(start, i - start) + " is too large");
    shape.push_back(std::stoll(h.substr(start, i - start)));
  }
  return shape;
}

inline std::string ShapeRepr(const std::vector<int64_t> &shape) {
  std::string s = "(";
  for (size_t i = 0; i < shape.size(); ++i) {
    if (i) s += ", ";
    s += std::to_string(shape[i]);
  }
  if (shape.size() == 1) s += ",";
  return s + ")";
}

}  // namespace detail

// Reads a C-order array; `want` (if non-empty) lists the accepted descrs.
inline Array Read(const std::string &path, const std::vector<std::string> &want = {}) {
  std::ifstream in(path, std::ios::binary);
  if (!in) throw Error("cannot open " + path);
  char magic[6];
  in.read(magic, 6);
  if (!in || std::memcmp(magic, "\x93NUMPY", 6) != 0) throw Error(path + " is not a .npy file");
  unsigned char ver[2];
  in.read(reinterpret_cast<char *>(ver), 2);
  uint64_t hlen = 0;
  if (ver[0] == 1) {
    unsigned char b[2];
    in.read(reinterpret_cast<char *>(b), 2);
    hlen = b[0] | (uint64_t)b[1] << 8;
  } else if (ver[0] == 2 || ver[0] == 3) {
    unsigned char b[4];
    in.read(reinterpret_cast<char *>(b), 4);
    hlen = b[0] | (uint64_t)b[1] << 8 | (uint64_t)b[2] << 16 | (uint64_t)b[3] << 24;
  } else {
    throw Error(path + ": unsupported .npy version " + std::to_string(ver[0]));
  }
  if (!in || hlen > (1u << 20)) throw Error(path + ": truncated .npy header");
  std::string h(hlen, '\0');
  in.read(h.data(), (std::streamsize)hlen);
  if (!in) throw Error(path + ": truncated .npy header");
  Array a;
  a.descr = detail::QuotedAfter(h, "'descr'");
  if (a.descr == "|V2") a.descr = "<V2";
  const size_t fo = h.find("'fortran_order'");
  if (fo != std::string::npos && h.find("True", fo) != std::string::npos && h.find("True", fo) < h.find(',', fo))
    throw Error(path + ": Fortran-order arrays are not supported");
  const int isz = ItemSize(a.descr);
  if (isz == 0) throw Error(path + ": unsupported dtype '" + a.descr + "'");
  if (!want.empty()) {
    bool ok = false;
    for (const std::string &w : want) ok = ok || w == a.descr;
    if (!ok) throw Error(path + ": dtype '" + a.descr + "' where " + want[0] + " was expected");
  }
  a.shape = detail::Shape(h);
  // the payload's size, checked for overflow, against what the file holds
  // before anything is allocated
  uint64_t bytes = (uint64_t)isz;
  for (int64_t d : a.shape) {
    if (d < 0) throw Error(path + ": negative dimension");
    if (d != 0 && bytes > (uint64_t(1) << 62) / (uint64_t)d)
      throw Error(path + ": shape " + detail::ShapeRepr(a.shape) + " is too large");
    bytes *= (uint64_t)d;
  }
  const std::streampos here = in.tellg();
  in.seekg(0, std::ios::end);
  const std::streampos end = in.tellg();
  in.seekg(here);
  if (!in || here < 0 || end < here || (uint64_t)(end - here) < bytes)
    throw Error(path + ": truncated .npy payload (shape " + detail::ShapeRepr(a.shape) + " needs " + std::to_string(bytes) +
                " bytes)");
  a.data.resize((size_t)bytes);
  in.read(reinterpret_cast<char *>(a.data.data()), (std::streamsize)a.data.size());
  if (!in) throw Error(path + ": truncated .npy payload");
  return a;
}

inline void Write(const std::string &path, const std::string &descr, const std::vector<int64_t> &shape,
                  const void *data) {
  const int isz = ItemSize(descr);
  if (isz == 0) throw Error("npy write: unsupported dtype " + descr);
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  const std::string dict =
      "{'descr': '" + descr + "', 'fortran_order': False, 'shape': " + detail::ShapeRepr(shape) + ", }";
  const size_t prefix = 10;  // magic, version, 2-byte length
  const size_t total = ((prefix + dict.size() + 1 + 63) / 64) * 64;
  std::string header = dict;
  header.append(total - prefix - dict.size() - 1, ' ');
  header.push_back('\n');
  std::ofstream out(path, std::ios::binary | std::ios::trunc);
  if (!out) throw Error("cannot open " + path + " for writing");
  out.write("\x93NUMPY", 6);
  const unsigned char ver[2] = {1, 0};
  out.write(reinterpret_cast<const char *>(ver), 2);
  const unsigned char len[2] = {(unsigned char)(header.size() & 0xFF), (unsigned char)(header.size() >> 8)};
  out.write(reinterpret_cast<const char *>(len), 2);
  out.write(header.data(), (std::streamsize)header.size());
  out.write(static_cast<const char *>(data), (std::streamsize)(n * isz));
  if (!out) throw Error("failed writing " + path);
}

}  // namespace pk::npy
