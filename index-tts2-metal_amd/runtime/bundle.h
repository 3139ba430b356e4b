// bundle.h -- MIT2 weight bundle: mmap loader and writer.
//
// Same interface and on-disk format as the reference's loader
// (runtime/include/mit2/bundle.hpp:11-79, runtime/bundle.cpp; format in
// docs/native_bundle.md):
//   manifest.json  {"format":"MIT2","version":1,"endianness":"little",
//                   "alignment":A,"weights_file":"weights.bin",
//                   "tensors":[{"name","shape","dtype","offset","nbytes",
//                               "sha256","layout","component"}, ...]}
//   weights.bin    "MIT2" u32 version u32 alignment, then each payload at an
//                  A-aligned offset.
// A single-file bundle (payloads, then the manifest, then a 24-byte footer
// [u64 manifest_offset][u64 manifest_size]["MIT2VOIC"]) is accepted too.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

namespace mit2 {

struct TensorInfo {
  std::string name;
  std::vector<int64_t> shape;
  std::string dtype;  // f32 f16 i64 i32 u32 u8
  uint64_t offset = 0;
  uint64_t nbytes = 0;
  std::string sha256;
  std::string layout;
  std::string component;
};

class MappedFile {
 public:
  MappedFile() = default;
  explicit MappedFile(const std::string& path);
  ~MappedFile();
  MappedFile(const MappedFile&) = delete;
  MappedFile& operator=(const MappedFile&) = delete;
  MappedFile(MappedFile&& o) noexcept;
  MappedFile& operator=(MappedFile&& o) noexcept;
  const uint8_t* data() const { return static_cast<const uint8_t*>(data_); }
  size_t size() const { return size_; }
  bool valid() const { return data_ != nullptr; }

 private:
  void release();
  int fd_ = -1;
  void* data_ = nullptr;
  size_t size_ = 0;
};

bool bundle_path_is_single_file(const std::string& path);

class Bundle {
 public:
  // Opens a bundle directory or a single-file bundle.  Throws
  // std::runtime_error on any violation of the format's validation rules.
  explicit Bundle(const std::string& path);

  const std::vector<TensorInfo>& tensors() const { return d_->tensors; }
  const TensorInfo* find(const std::string& name) const;
  const uint8_t* tensor_data(const TensorInfo& info) const;
  size_t tensor_count() const { return d_->tensors.size(); }
  size_t total_tensor_bytes() const;
  const std::string& root() const { return d_->root; }
  const std::string& weights_file() const { return d_->weights_file; }
  size_t weights_size() const { return d_->weights.size(); }
  uint32_t version() const { return d_->version; }
  uint32_t alignment() const { return d_->alignment; }
  const std::string& endianness() const { return d_->endianness; }

  struct Data {
    std::string root;
    std::string weights_file;
    uint32_t version = 0;
    uint32_t alignment = 0;
    std::string endianness;
    MappedFile weights;
    std::vector<TensorInfo> tensors;
    std::unordered_map<std::string, size_t> by_name;
  };

 private:
  std::shared_ptr<Data> d_;
};

// Bytes per element of a bundle dtype (0 for an unknown dtype).
size_t dtype_size(const std::string& dtype);

// Payload for write_bundle.
struct TensorPayload {
  std::string name;
  std::vector<int64_t> shape;
  std::string dtype;
  std::string component;
  std::vector<uint8_t> bytes;
};

// Writes dir/manifest.json and dir/weights.bin (alignment 4096, SHA-256 of
// every payload recorded).  Throws std::runtime_error on I/O failure.
void write_bundle(const std::string& dir, const std::vector<TensorPayload>& tensors);

// SHA-256 of a byte range, lowercase hex.
std::string sha256_hex(const uint8_t* data, size_t n);

}  // namespace mit2
