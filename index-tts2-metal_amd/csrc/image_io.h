// image_io.h -- byte-level helpers of the device weight image (a file that
// holds the prepared device weights so that a context is created by copying
// them, with no host-side preparation).
#pragma once

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace mit2hip {

// Appends plain values to an image buffer.
struct ImageWriter {
  std::vector<uint8_t>& out;
  template <typename T>
  void put(const T& v) {
    const size_t n = out.size();
    out.resize(n + sizeof(T));
    std::memcpy(out.data() + n, &v, sizeof(T));
  }
  void bytes(const void* p, size_t n) {
    const size_t at = out.size();
    out.resize(at + n);
    std::memcpy(out.data() + at, p, n);
  }
};

// Reads plain values from an image buffer; every read is bounds-checked and
// a short image is a model error.
struct ImageReader {
  const uint8_t* p;
  size_t n;
  size_t at = 0;
  template <typename T>
  T get() {
    T v;
    need(sizeof(T));
    std::memcpy(&v, p + at, sizeof(T));
    at += sizeof(T);
    return v;
  }
  const uint8_t* bytes(size_t k) {
    need(k);
    const uint8_t* q = p + at;
    at += k;
    return q;
  }
  void need(size_t k) const {
    if (k > n - at) throw std::runtime_error("device image: truncated or malformed");
  }
};

// Offset of a device pointer inside an arena (UINT64_MAX for null), and back.
inline uint64_t arena_offset(const void* ptr, const char* base) {
  return ptr ? (uint64_t)(static_cast<const char*>(ptr) - base) : UINT64_MAX;
}
template <typename T>
inline T* arena_pointer(uint64_t off, char* base, size_t used) {
  if (off == UINT64_MAX) return nullptr;
  if (off >= used) throw std::runtime_error("device image: pointer outside its arena");
  return reinterpret_cast<T*>(base + off);
}

// A device array of `count` T at arena offset `off`, checked to lie inside
// the arena's used bytes.
template <typename T>
inline T* arena_span(uint64_t off, size_t count, char* base, size_t used) {
  if (off == UINT64_MAX || off > used || count * sizeof(T) > used - off)
    throw std::runtime_error("device image: array outside its arena");
  return reinterpret_cast<T*>(base + off);
}

// 64-bit FNV-1a over 8-byte words (and the tail bytes): a fast integrity
// check of the image payload.
inline uint64_t image_checksum(const uint8_t* p, size_t n) {
  uint64_t h = 0xcbf29ce484222325ull;
  size_t i = 0;
  for (; i + 8 <= n; i += 8) {
    uint64_t w;
    std::memcpy(&w, p + i, 8);
    h = (h ^ w) * 0x100000001b3ull;
  }
  for (; i < n; ++i) h = (h ^ p[i]) * 0x100000001b3ull;
  return h;
}

}  // namespace mit2hip
