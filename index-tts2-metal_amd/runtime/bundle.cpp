// bundle.cpp -- MIT2 bundle loader / writer (format: docs/native_bundle.md of
// the reference; interface: runtime/include/mit2/bundle.hpp).
//
// The manifest is read with a small recursive-descent JSON parser (the
// reference matches keys with regular expressions); every rule listed in the
// format's "Validation Rules" that applies to a weights bundle is enforced:
// format/version/endianness, weights.bin header magic/version/alignment,
// duplicate names, zero-byte tensors, unaligned offsets, payloads past the end
// of the file, dtype x shape byte-count mismatches and overlapping payloads.
#include "bundle.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <cstring>
#include <fstream>
#include <map>
#include <sstream>
#include <stdexcept>

namespace mit2 {

// ------------------------------------------------------------------ mmap
MappedFile::MappedFile(const std::string& path) {
  fd_ = ::open(path.c_str(), O_RDONLY);
  if (fd_ < 0) throw std::runtime_error("failed to open mapped file: " + path);
  struct stat st {};
  if (fstat(fd_, &st) != 0) {
    release();
    throw std::runtime_error("failed to stat mapped file: " + path);
  }
  size_ = static_cast<size_t>(st.st_size);
  if (size_ == 0) {
    release();
    throw std::runtime_error("mapped file is empty: " + path);
  }
  data_ = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
  if (data_ == MAP_FAILED) {
    data_ = nullptr;
    release();
    throw std::runtime_error("failed to mmap file: " + path);
  }
}

void MappedFile::release() {
  if (data_) munmap(data_, size_);
  if (fd_ >= 0) ::close(fd_);
  data_ = nullptr;
  fd_ = -1;
  size_ = 0;
}

MappedFile::~MappedFile() { release(); }

MappedFile::MappedFile(MappedFile&& o) noexcept { *this = std::move(o); }

MappedFile& MappedFile::operator=(MappedFile&& o) noexcept {
  if (this != &o) {
    release();
    fd_ = o.fd_;
    data_ = o.data_;
    size_ = o.size_;
    o.fd_ = -1;
    o.data_ = nullptr;
    o.size_ = 0;
  }
  return *this;
}

// ------------------------------------------------------------------ JSON
namespace {

struct JValue {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0;
  std::string numtext;
  std::string str;
  std::vector<JValue> arr;
  std::vector<std::pair<std::string, JValue>> obj;
  const JValue* get(const std::string& key) const {
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

class JParser {
 public:
  explicit JParser(const std::string& s) : s_(s) {}
  JValue parse() {
    JValue v = value();
    ws();
    if (i_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void fail(const char* what) {
    throw std::runtime_error(std::string("manifest JSON: ") + what + " at offset " +
                             std::to_string(i_));
  }
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t'))
      ++i_;
  }
  bool eat(char c) {
    ws();
    if (i_ < s_.size() && s_[i_] == c) {
      ++i_;
      return true;
    }
    return false;
  }
  JValue value() {
    ws();
    if (i_ >= s_.size()) fail("unexpected end");
    const char c = s_[i_];
    JValue v;
    if (c == '{') {
      ++i_;
      v.kind = JValue::Obj;
      if (eat('}')) return v;
      do {
        ws();
        if (i_ >= s_.size() || s_[i_] != '"') fail("expected key");
        std::string k = string();
        if (!eat(':')) fail("expected ':'");
        v.obj.emplace_back(std::move(k), value());
      } while (eat(','));
      if (!eat('}')) fail("expected '}'");
    } else if (c == '[') {
      ++i_;
      v.kind = JValue::Arr;
      if (eat(']')) return v;
      do {
        v.arr.push_back(value());
      } while (eat(','));
      if (!eat(']')) fail("expected ']'");
    } else if (c == '"') {
      v.kind = JValue::Str;
      v.str = string();
    } else if (s_.compare(i_, 4, "true") == 0) {
      i_ += 4;
      v.kind = JValue::Bool;
      v.b = true;
    } else if (s_.compare(i_, 5, "false") == 0) {
      i_ += 5;
      v.kind = JValue::Bool;
    } else if (s_.compare(i_, 4, "null") == 0) {
      i_ += 4;
    } else {
      const size_t st = i_;
      while (i_ < s_.size() && (std::isdigit((unsigned char)s_[i_]) || s_[i_] == '-' ||
                                s_[i_] == '+' || s_[i_] == '.' || s_[i_] == 'e' || s_[i_] == 'E'))
        ++i_;
      if (st == i_) fail("unexpected character");
      v.kind = JValue::Num;
      v.numtext = s_.substr(st, i_ - st);
      v.num = std::stod(v.numtext);
    }
    return v;
  }
  std::string string() {
    ++i_;  // opening quote
    std::string out;
    while (i_ < s_.size() && s_[i_] != '"') {
      char c = s_[i_++];
      if (c == '\\') {
        if (i_ >= s_.size()) fail("bad escape");
        const char e = s_[i_++];
        switch (e) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {
            if (i_ + 4 > s_.size()) fail("bad \\u escape");
            const unsigned cp = std::stoul(s_.substr(i_, 4), nullptr, 16);
            i_ += 4;
            if (cp < 0x80) {
              out += (char)cp;
            } else if (cp < 0x800) {
              out += (char)(0xC0 | (cp >> 6));
              out += (char)(0x80 | (cp & 0x3F));
            } else {
              out += (char)(0xE0 | (cp >> 12));
              out += (char)(0x80 | ((cp >> 6) & 0x3F));
              out += (char)(0x80 | (cp & 0x3F));
            }
            break;
          }
          default: fail("bad escape");
        }
      } else {
        out += c;
      }
    }
    if (i_ >= s_.size()) fail("unterminated string");
    ++i_;
    return out;
  }
  const std::string& s_;
  size_t i_ = 0;
};

std::string read_text(const std::string& path) {
  std::ifstream fp(path, std::ios::binary);
  if (!fp) throw std::runtime_error("failed to open " + path);
  std::ostringstream ss;
  ss << fp.rdbuf();
  return ss.str();
}

uint64_t as_u64(const JValue* v, const char* what) {
  if (!v || v->kind != JValue::Num || v->numtext.find_first_of(".eE-") != std::string::npos)
    throw std::runtime_error(std::string("manifest: ") + what + " must be a non-negative integer");
  return std::stoull(v->numtext);
}

std::string as_str(const JValue* v, const std::string& fallback) {
  if (!v) return fallback;
  if (v->kind != JValue::Str) throw std::runtime_error("manifest: expected a string value");
  return v->str;
}

uint32_t rd_u32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

uint64_t rd_u64(const uint8_t* p) {
  uint64_t v = 0;
  for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];
  return v;
}

constexpr char kFooterMagic[8] = {'M', 'I', 'T', '2', 'V', 'O', 'I', 'C'};
constexpr size_t kFooterSize = 24;

}  // namespace

size_t dtype_size(const std::string& d) {
  if (d == "f32" || d == "i32" || d == "u32") return 4;
  if (d == "f16") return 2;
  if (d == "i64") return 8;
  if (d == "u8") return 1;
  return 0;
}

bool bundle_path_is_single_file(const std::string& path) {
  struct stat st {};
  if (stat(path.c_str(), &st) != 0 || !S_ISREG(st.st_mode)) return false;
  std::ifstream fp(path, std::ios::binary);
  char magic[4] = {};
  fp.read(magic, 4);
  return fp && std::memcmp(magic, "MIT2", 4) == 0;
}

// ------------------------------------------------------------------ loader
Bundle::Bundle(const std::string& path) {
  d_ = std::make_shared<Data>();
  d_->root = path;
  struct stat st {};
  const bool single = stat(path.c_str(), &st) == 0 && S_ISREG(st.st_mode);
  std::string json;
  if (single) {
    d_->weights_file = path;
    d_->weights = MappedFile(path);
    if (d_->weights.size() < 12 + kFooterSize)
      throw std::runtime_error("single-file bundle is too small: " + path);
    const uint8_t* footer = d_->weights.data() + d_->weights.size() - kFooterSize;
    if (std::memcmp(footer + 16, kFooterMagic, 8) != 0)
      throw std::runtime_error("single-file bundle footer magic missing: " + path);
    const uint64_t mo = rd_u64(footer), ms = rd_u64(footer + 8);
    if (mo > d_->weights.size() - kFooterSize || ms > d_->weights.size() - kFooterSize - mo)
      throw std::runtime_error("single-file bundle manifest exceeds file: " + path);
    json.assign(reinterpret_cast<const char*>(d_->weights.data() + mo), (size_t)ms);
  } else {
    json = read_text(path + "/manifest.json");
  }
  const JValue root = JParser(json).parse();
  if (root.kind != JValue::Obj) throw std::runtime_error("manifest must be a JSON object");
  const std::string format = as_str(root.get("format"), "");
  if (format != "MIT2") throw std::runtime_error("unsupported bundle format: " + format);
  d_->version = (uint32_t)as_u64(root.get("version"), "version");
  d_->alignment = (uint32_t)as_u64(root.get("alignment"), "alignment");
  d_->endianness = as_str(root.get("endianness"), "");
  if (d_->version != 1)
    throw std::runtime_error("unsupported bundle version: " + std::to_string(d_->version));
  if (d_->alignment == 0) throw std::runtime_error("bundle alignment must be non-zero");
  if (d_->endianness != "little")
    throw std::runtime_error("unsupported bundle endianness: " + d_->endianness);
  if (!single) {
    d_->weights_file = as_str(root.get("weights_file"), "weights.bin");
    d_->weights = MappedFile(path + "/" + d_->weights_file);
  }
  if (d_->weights.size() < 12) throw std::runtime_error("weights file is too small for MIT2 header");
  const uint8_t* hdr = d_->weights.data();
  if (std::memcmp(hdr, "MIT2", 4) != 0) throw std::runtime_error("weights file has invalid MIT2 magic");
  if (rd_u32(hdr + 4) != d_->version) throw std::runtime_error("weights header version mismatch");
  if (rd_u32(hdr + 8) != d_->alignment) throw std::runtime_error("weights header alignment mismatch");

  const JValue* tensors = root.get("tensors");
  if (!tensors || tensors->kind != JValue::Arr) throw std::runtime_error("manifest missing tensors");
  for (const JValue& o : tensors->arr) {
    if (o.kind != JValue::Obj) throw std::runtime_error("tensor record must be an object");
    TensorInfo info;
    info.name = as_str(o.get("name"), "");
    if (info.name.empty()) throw std::runtime_error("tensor record has empty name");
    const JValue* shape = o.get("shape");
    if (!shape || shape->kind != JValue::Arr) throw std::runtime_error("missing tensor shape: " + info.name);
    for (const JValue& d : shape->arr) info.shape.push_back((int64_t)as_u64(&d, "shape entry"));
    info.dtype = as_str(o.get("dtype"), "");
    info.offset = as_u64(o.get("offset"), "offset");
    info.nbytes = as_u64(o.get("nbytes"), "nbytes");
    info.sha256 = as_str(o.get("sha256"), "");
    info.layout = as_str(o.get("layout"), "row_major");
    info.component = as_str(o.get("component"), "unknown");
    if (d_->by_name.count(info.name)) throw std::runtime_error("duplicate tensor in manifest: " + info.name);
    if (info.offset % d_->alignment != 0)
      throw std::runtime_error("tensor offset is not bundle-aligned: " + info.name);
    if (info.nbytes == 0) throw std::runtime_error("tensor has zero bytes: " + info.name);
    if (info.offset > d_->weights.size() || info.nbytes > d_->weights.size() - info.offset)
      throw std::runtime_error("tensor extends beyond weights file: " + info.name);
    const size_t es = dtype_size(info.dtype);
    if (es == 0) throw std::runtime_error("unsupported dtype " + info.dtype + ": " + info.name);
    uint64_t count = 1;
    for (int64_t dim : info.shape) count *= (uint64_t)dim;
    if (count * es != info.nbytes)
      throw std::runtime_error("dtype/shape byte count mismatch: " + info.name);
    d_->by_name[info.name] = d_->tensors.size();
    d_->tensors.push_back(std::move(info));
  }
  // Payload ranges must not overlap (and must not overlap the 12-byte header).
  std::vector<std::pair<uint64_t, uint64_t>> ranges;
  for (const auto& t : d_->tensors) ranges.emplace_back(t.offset, t.offset + t.nbytes);
  std::sort(ranges.begin(), ranges.end());
  uint64_t end = 12;
  for (const auto& r : ranges) {
    if (r.first < end) throw std::runtime_error("overlapping tensor payload ranges");
    end = r.second;
  }
}

const TensorInfo* Bundle::find(const std::string& name) const {
  auto it = d_->by_name.find(name);
  return it == d_->by_name.end() ? nullptr : &d_->tensors[it->second];
}

const uint8_t* Bundle::tensor_data(const TensorInfo& info) const {
  return d_->weights.data() + info.offset;
}

size_t Bundle::total_tensor_bytes() const {
  size_t n = 0;
  for (const auto& t : d_->tensors) n += (size_t)t.nbytes;
  return n;
}

// ------------------------------------------------------------------ SHA-256 (FIPS 180-4)
namespace {
constexpr uint32_t kK[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

void sha_block(uint32_t h[8], const uint8_t* p) {
  uint32_t w[64];
  for (int i = 0; i < 16; ++i)
    w[i] = ((uint32_t)p[4 * i] << 24) | ((uint32_t)p[4 * i + 1] << 16) | ((uint32_t)p[4 * i + 2] << 8) |
           p[4 * i + 3];
  for (int i = 16; i < 64; ++i) {
    const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
    const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
    w[i] = w[i - 16] + s0 + w[i - 7] + s1;
  }
  uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
  for (int i = 0; i < 64; ++i) {
    const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
    const uint32_t ch = (e & f) ^ (~e & g);
    const uint32_t t1 = hh + S1 + ch + kK[i] + w[i];
    const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
    const uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
    const uint32_t t2 = S0 + mj;
    hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
  }
  h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
}
}  // namespace

std::string sha256_hex(const uint8_t* data, size_t n) {
  uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                   0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
  size_t i = 0;
  for (; i + 64 <= n; i += 64) sha_block(h, data + i);
  uint8_t tail[128] = {};
  const size_t rem = n - i;
  std::memcpy(tail, data + i, rem);
  tail[rem] = 0x80;
  const size_t tl = rem + 9 <= 64 ? 64 : 128;
  const uint64_t bits = (uint64_t)n * 8;
  for (int k = 0; k < 8; ++k) tail[tl - 1 - k] = (uint8_t)(bits >> (8 * k));
  sha_block(h, tail);
  if (tl == 128) sha_block(h, tail + 64);
  static const char* hex = "0123456789abcdef";
  std::string out(64, '0');
  for (int k = 0; k < 8; ++k)
    for (int j = 0; j < 4; ++j) {
      const uint8_t byte = (uint8_t)(h[k] >> (24 - 8 * j));
      out[k * 8 + j * 2] = hex[byte >> 4];
      out[k * 8 + j * 2 + 1] = hex[byte & 15];
    }
  return out;
}

// ------------------------------------------------------------------ writer
void write_bundle(const std::string& dir, const std::vector<TensorPayload>& tensors) {
  constexpr uint64_t kAlign = 4096;
  ::mkdir(dir.c_str(), 0755);
  std::ofstream w(dir + "/weights.bin", std::ios::binary | std::ios::trunc);
  if (!w) throw std::runtime_error("cannot write " + dir + "/weights.bin");
  const uint8_t hdr[12] = {'M', 'I', 'T', '2', 1, 0, 0, 0, (uint8_t)(kAlign & 0xff),
                           (uint8_t)((kAlign >> 8) & 0xff), 0, 0};
  w.write(reinterpret_cast<const char*>(hdr), 12);
  uint64_t pos = 12;
  std::ostringstream m;
  m << "{\n  \"alignment\": " << kAlign << ",\n  \"endianness\": \"little\",\n"
    << "  \"format\": \"MIT2\",\n  \"metadata\": {},\n  \"tensors\": [";
  static const std::vector<char> zeros(kAlign, 0);
  for (size_t i = 0; i < tensors.size(); ++i) {
    const auto& t = tensors[i];
    const uint64_t off = (pos + kAlign - 1) / kAlign * kAlign;
    w.write(zeros.data(), (std::streamsize)(off - pos));
    w.write(reinterpret_cast<const char*>(t.bytes.data()), (std::streamsize)t.bytes.size());
    pos = off + t.bytes.size();
    m << (i ? ",\n" : "\n") << "    {\"component\": \"" << t.component << "\", \"dtype\": \""
      << t.dtype << "\", \"layout\": \"row_major\", \"name\": \"" << t.name
      << "\", \"nbytes\": " << t.bytes.size() << ", \"offset\": " << off << ", \"sha256\": \""
      << sha256_hex(t.bytes.data(), t.bytes.size()) << "\", \"shape\": [";
    for (size_t d = 0; d < t.shape.size(); ++d) m << (d ? ", " : "") << t.shape[d];
    m << "]}";
  }
  m << "\n  ],\n  \"version\": 1,\n  \"weights_file\": \"weights.bin\"\n}\n";
  if (!w) throw std::runtime_error("write failed: " + dir + "/weights.bin");
  w.close();
  std::ofstream mf(dir + "/manifest.json", std::ios::trunc);
  mf << m.str();
  if (!mf) throw std::runtime_error("cannot write " + dir + "/manifest.json");
}

}  // namespace mit2
