// Resident MXFP4 weights on disk and their SafeTensors sources (host code).
//
// - GOSSMX4 repack containers as CpuRepackCache writes and reads them
//   (crates/gpt-oss-model-runner/src/cpu_repack.rs:21-23, 92-130, 149-330,
//   400-480), for the reference's layouts 1 and 2 and this library's resident
//   layout 3 (GpuTiledV3);
// - SafeTensors shards as CpuTensorStore parses them (cpu_tensor_store.rs:
//   46-98, 176-288);
// - CpuRepackCache::open_or_create with layout 3: cache key, lock file,
//   atomic publish.
// SHA-256 follows FIPS 180-4; JSON is read and written by the small codec
// below (RFC 8259 values; the writer emits serde_json's compact form).

#include "../../include/gossmx.h"
#include "gossmx_internal.h"

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <fcntl.h>
#include <string>
#include <sys/stat.h>
#include <thread>
#include <unistd.h>
#include <utility>
#include <vector>

namespace {

constexpr char kMagic[8] = {'G', 'O', 'S', 'S', 'M', 'X', '4', '\0'};
constexpr uint32_t kFormatVersion = 1;  // REPACK_FORMAT_VERSION
constexpr size_t kRecordBytes = 17;
constexpr size_t kMaxHeaderBytes = 64u << 20;
constexpr int kMaxJsonDepth = 64;

int err(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return gossmx::set_error(status, buf);
}

const char* layout_name(int layout) {
  switch (layout) {
    case GOSSMX_LAYOUT_CANONICAL_V1: return "CanonicalAdjacentV1";
    case GOSSMX_LAYOUT_X8_SPLIT_V2: return "InterleavedSplitX8V2";
    case GOSSMX_LAYOUT_GPU_TILED_V3: return "GpuTiledV3";
    default: return nullptr;
  }
}

// ---------------------------------------------------------------------------
// SHA-256 (FIPS 180-4, section 6.2).

class Sha256 {
 public:
  Sha256() {
    static const uint32_t init[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                                     0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    std::memcpy(h_, init, sizeof h_);
  }
  void update(const void* data, size_t n) {
    const uint8_t* p = static_cast<const uint8_t*>(data);
    total_ += n;
    while (n > 0) {
      const size_t take = std::min(n, sizeof buf_ - used_);
      std::memcpy(buf_ + used_, p, take);
      used_ += take;
      p += take;
      n -= take;
      if (used_ == sizeof buf_) {
        block(buf_);
        used_ = 0;
      }
    }
  }
  void hex(char out[65]) {
    const uint64_t bits = total_ * 8;
    const uint8_t one = 0x80, zero = 0;
    update(&one, 1);
    while (used_ != 56) update(&zero, 1);
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
    update(len, 8);
    static const char digits[] = "0123456789abcdef";
    for (int i = 0; i < 8; ++i)
      for (int j = 0; j < 4; ++j) {
        const uint8_t b = (uint8_t)(h_[i] >> (24 - 8 * j));
        out[8 * i + 2 * j] = digits[b >> 4];
        out[8 * i + 2 * j + 1] = digits[b & 15];
      }
    out[64] = '\0';
  }

 private:
  static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
  void block(const uint8_t* b) {
    static const uint32_t k[64] = {
        0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
        0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
        0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
        0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
        0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
        0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
        0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
        0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};
    uint32_t w[64];
    for (int t = 0; t < 16; ++t)
      w[t] = (uint32_t)b[4 * t] << 24 | (uint32_t)b[4 * t + 1] << 16 | (uint32_t)b[4 * t + 2] << 8 | b[4 * t + 3];
    for (int t = 16; t < 64; ++t) {
      const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
      const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
      w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t a = h_[0], bb = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], h = h_[7];
    for (int t = 0; t < 64; ++t) {
      const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[t] + w[t];
      const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & bb) ^ (a & c) ^ (bb & c));
      h = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = bb;
      bb = a;
      a = t1 + t2;
    }
    h_[0] += a;
    h_[1] += bb;
    h_[2] += c;
    h_[3] += d;
    h_[4] += e;
    h_[5] += f;
    h_[6] += g;
    h_[7] += h;
  }
  uint32_t h_[8];
  uint8_t buf_[64];
  size_t used_ = 0;
  uint64_t total_ = 0;
};

// ---------------------------------------------------------------------------
// JSON values (RFC 8259). Numbers keep their exact unsigned value when they
// are non-negative integers.

struct Json {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
  bool boolean = false;
  bool is_uint = false;
  uint64_t uint = 0;
  std::string str;
  std::vector<Json> items;
  std::vector<std::pair<std::string, Json>> members;

  const Json* get(const char* key) const {
    for (const auto& m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
};

class JsonReader {
 public:
  JsonReader(const char* p, size_t n) : p_(p), end_(p + n) {}
  bool parse(Json& out) {
    if (!value(out, 0)) return false;
    ws();
    return p_ == end_;
  }

 private:
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if ((size_t)(end_ - p_) < n || std::memcmp(p_, s, n) != 0) return false;
    p_ += n;
    return true;
  }
  static void utf8(std::string& s, uint32_t c) {
    if (c < 0x80) {
      s += (char)c;
    } else if (c < 0x800) {
      s += (char)(0xC0 | (c >> 6));
      s += (char)(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      s += (char)(0xE0 | (c >> 12));
      s += (char)(0x80 | ((c >> 6) & 0x3F));
      s += (char)(0x80 | (c & 0x3F));
    } else {
      s += (char)(0xF0 | (c >> 18));
      s += (char)(0x80 | ((c >> 12) & 0x3F));
      s += (char)(0x80 | ((c >> 6) & 0x3F));
      s += (char)(0x80 | (c & 0x3F));
    }
  }
  bool hex4(uint32_t& v) {
    if (end_ - p_ < 4) return false;
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  // One UTF-8 sequence in a string's raw bytes, from its lead byte c (the
  // input must be valid UTF-8, as serde_json::from_slice requires: no
  // overlong forms, no surrogates, nothing above U+10FFFF).
  bool raw_utf8(std::string& s, unsigned char c) {
    int n;
    uint32_t cp, min;
    if (c >= 0xC2 && c <= 0xDF) n = 1, cp = c & 0x1F, min = 0x80;
    else if (c >= 0xE0 && c <= 0xEF) n = 2, cp = c & 0x0F, min = 0x800;
    else if (c >= 0xF0 && c <= 0xF4) n = 3, cp = c & 0x07, min = 0x10000;
    else return false;
    if (end_ - p_ < n) return false;
    for (int i = 0; i < n; ++i) {
      const unsigned char b = (unsigned char)p_[i];
      if ((b & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (b & 0x3F);
    }
    if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp < 0xE000)) return false;
    s += (char)c;
    s.append(p_, (size_t)n);
    p_ += n;
    return true;
  }
  bool string(std::string& s) {
    if (p_ >= end_ || *p_ != '"') return false;
    ++p_;
    while (p_ < end_) {
      const char c = *p_++;
      if (c == '"') return true;
      if ((unsigned char)c < 0x20) return false;
      if ((unsigned char)c >= 0x80) {
        if (!raw_utf8(s, (unsigned char)c)) return false;
        continue;
      }
      if (c != '\\') {
        s += c;
        continue;
      }
      if (p_ >= end_) return false;
      const char e = *p_++;
      switch (e) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t c1;
          if (!hex4(c1)) return false;
          if (c1 >= 0xD800 && c1 < 0xDC00) {
            uint32_t c2;
            if (!lit("\\u") || !hex4(c2) || c2 < 0xDC00 || c2 >= 0xE000) return false;
            c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
          } else if (c1 >= 0xDC00 && c1 < 0xE000) {
            return false;
          }
          utf8(s, c1);
          break;
        }
        default: return false;
      }
    }
    return false;
  }
  bool number(Json& v) {
    const char* start = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
    if (*p_ == '0') ++p_;
    else while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    bool integral = true;
    if (p_ < end_ && *p_ == '.') {
      integral = false;
      ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      integral = false;
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    v.kind = Json::kNumber;
    if (integral && *start != '-') {
      uint64_t u = 0;
      for (const char* q = start; q < p_; ++q) {
        const uint64_t d = (uint64_t)(*q - '0');
        if (u > (UINT64_MAX - d) / 10) return true;  // out of u64 range: not an exact uint
        u = u * 10 + d;
      }
      v.is_uint = true;
      v.uint = u;
    }
    return true;
  }
  bool value(Json& v, int depth) {
    if (depth > kMaxJsonDepth) return false;
    ws();
    if (p_ >= end_) return false;
    const char c = *p_;
    if (c == '{') {
      ++p_;
      v.kind = Json::kObject;
      ws();
      if (p_ < end_ && *p_ == '}') {
        ++p_;
        return true;
      }
      while (true) {
        ws();
        std::pair<std::string, Json> m;
        if (!string(m.first)) return false;
        ws();
        if (p_ >= end_ || *p_++ != ':') return false;
        if (!value(m.second, depth + 1)) return false;
        v.members.push_back(std::move(m));
        ws();
        if (p_ >= end_) return false;
        if (*p_ == ',') {
          ++p_;
          continue;
        }
        if (*p_++ == '}') return true;
        return false;
      }
    }
    if (c == '[') {
      ++p_;
      v.kind = Json::kArray;
      ws();
      if (p_ < end_ && *p_ == ']') {
        ++p_;
        return true;
      }
      while (true) {
        Json item;
        if (!value(item, depth + 1)) return false;
        v.items.push_back(std::move(item));
        ws();
        if (p_ >= end_) return false;
        if (*p_ == ',') {
          ++p_;
          continue;
        }
        if (*p_++ == ']') return true;
        return false;
      }
    }
    if (c == '"') {
      v.kind = Json::kString;
      return string(v.str);
    }
    if (lit("true")) {
      v.kind = Json::kBool;
      v.boolean = true;
      return true;
    }
    if (lit("false")) {
      v.kind = Json::kBool;
      return true;
    }
    if (lit("null")) return true;
    return number(v);
  }
  const char* p_;
  const char* end_;
};

// serde_json's string escaping: '"', '\\' and control characters (the short
// escapes for \b \t \n \f \r, \u00xx in lowercase hex for the rest).
void json_string(std::string& out, const std::string& s) {
  static const char digits[] = "0123456789abcdef";
  out += '"';
  for (const char ch : s) {
    const unsigned char c = (unsigned char)ch;
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\b': out += "\\b"; break;
      case '\t': out += "\\t"; break;
      case '\n': out += "\\n"; break;
      case '\f': out += "\\f"; break;
      case '\r': out += "\\r"; break;
      default:
        if (c < 0x20) {
          out += "\\u00";
          out += digits[c >> 4];
          out += digits[c & 15];
        } else {
          out += (char)c;
        }
    }
  }
  out += '"';
}

// ---------------------------------------------------------------------------
// RepackHeader (cpu_repack.rs:120-130), in its serialized field order.

struct RepackHeader {
  uint32_t format_version = kFormatVersion;
  uint32_t layout_version = 0;
  std::string layout_identifier, tensor_name, model_revision;
  std::vector<std::string> source_hashes;
  size_t shape[3] = {0, 0, 0};
  size_t records = 0;

  bool operator==(const RepackHeader& o) const {
    return format_version == o.format_version && layout_version == o.layout_version &&
           layout_identifier == o.layout_identifier && tensor_name == o.tensor_name &&
           model_revision == o.model_revision && source_hashes == o.source_hashes && shape[0] == o.shape[0] &&
           shape[1] == o.shape[1] && shape[2] == o.shape[2] && records == o.records;
  }

  std::string serialize() const {
    std::string s = "{\"format_version\":" + std::to_string(format_version) +
                    ",\"layout_version\":" + std::to_string(layout_version) + ",\"layout_identifier\":";
    json_string(s, layout_identifier);
    s += ",\"tensor_name\":";
    json_string(s, tensor_name);
    s += ",\"model_revision\":";
    json_string(s, model_revision);
    s += ",\"source_hashes\":[";
    for (size_t i = 0; i < source_hashes.size(); ++i) {
      if (i) s += ',';
      json_string(s, source_hashes[i]);
    }
    s += "],\"shape\":[" + std::to_string(shape[0]) + "," + std::to_string(shape[1]) + "," + std::to_string(shape[2]) +
         "],\"records\":" + std::to_string(records) + "}";
    return s;
  }

  // Field-by-field deserialization with the types serde derives; unknown
  // fields are ignored, as serde does by default.
  bool parse(const Json& j) {
    if (j.kind != Json::kObject) return false;
    const Json* f;
    auto u = [](const Json* v, uint64_t max, uint64_t& out) {
      if (!v || v->kind != Json::kNumber || !v->is_uint || v->uint > max) return false;
      out = v->uint;
      return true;
    };
    auto str = [](const Json* v, std::string& out) {
      if (!v || v->kind != Json::kString) return false;
      out = v->str;
      return true;
    };
    uint64_t t;
    if (!u(j.get("format_version"), UINT32_MAX, t)) return false;
    format_version = (uint32_t)t;
    if (!u(j.get("layout_version"), UINT32_MAX, t)) return false;
    layout_version = (uint32_t)t;
    if (!str(j.get("layout_identifier"), layout_identifier) || !str(j.get("tensor_name"), tensor_name) ||
        !str(j.get("model_revision"), model_revision))
      return false;
    f = j.get("source_hashes");
    if (!f || f->kind != Json::kArray) return false;
    source_hashes.clear();
    for (const Json& h : f->items) {
      if (h.kind != Json::kString) return false;
      source_hashes.push_back(h.str);
    }
    f = j.get("shape");
    if (!f || f->kind != Json::kArray || f->items.size() != 3) return false;
    for (int i = 0; i < 3; ++i) {
      if (!u(&f->items[i], SIZE_MAX, t)) return false;
      shape[i] = (size_t)t;
    }
    if (!u(j.get("records"), SIZE_MAX, t)) return false;
    records = (size_t)t;
    return true;
  }
};

// ---------------------------------------------------------------------------
// Files.

struct File {
  int fd = -1;
  ~File() {
    if (fd >= 0) ::close(fd);
  }
};

int read_exact(int fd, void* dst, size_t n, size_t offset, const char* path) {
  uint8_t* p = static_cast<uint8_t*>(dst);
  while (n > 0) {
    const ssize_t r = ::pread(fd, p, n, (off_t)offset);
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return err(GOSSMX_ERR_BAD_FILE, "read of %s failed: %s", path, r < 0 ? strerror(errno) : "short file");
    p += r;
    n -= (size_t)r;
    offset += (size_t)r;
  }
  return GOSSMX_OK;
}

int write_all(int fd, const void* src, size_t n, const char* path) {
  const uint8_t* p = static_cast<const uint8_t*>(src);
  while (n > 0) {
    const ssize_t r = ::write(fd, p, n);
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return err(GOSSMX_ERR_BAD_FILE, "write of %s failed: %s", path, strerror(errno));
    p += r;
    n -= (size_t)r;
  }
  return GOSSMX_OK;
}

int open_read(const char* path, File& f, size_t& size) {
  f.fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (f.fd < 0) return err(GOSSMX_ERR_BAD_FILE, "cannot open %s: %s", path, strerror(errno));
  struct stat st;
  if (::fstat(f.fd, &st) != 0) return err(GOSSMX_ERR_BAD_FILE, "cannot stat %s: %s", path, strerror(errno));
  size = (size_t)st.st_size;
  return GOSSMX_OK;
}

std::string parent_dir(const std::string& path) {
  const size_t slash = path.rfind('/');
  if (slash == std::string::npos) return ".";
  if (slash == 0) return "/";
  return path.substr(0, slash);
}

int sync_directory(const std::string& dir) {
  const int fd = ::open(dir.c_str(), O_RDONLY | O_DIRECTORY | O_CLOEXEC);
  if (fd < 0) return err(GOSSMX_ERR_BAD_FILE, "cannot open directory %s: %s", dir.c_str(), strerror(errno));
  const int r = ::fsync(fd);
  ::close(fd);
  if (r != 0) return err(GOSSMX_ERR_BAD_FILE, "fsync of %s failed: %s", dir.c_str(), strerror(errno));
  return GOSSMX_OK;
}

int make_dirs(const std::string& dir) {
  std::string cur;
  size_t pos = 0;
  while (pos <= dir.size()) {
    const size_t next = dir.find('/', pos);
    cur = dir.substr(0, next == std::string::npos ? dir.size() : next);
    if (!cur.empty() && ::mkdir(cur.c_str(), 0755) != 0 && errno != EEXIST)
      return err(GOSSMX_ERR_BAD_FILE, "cannot create directory %s: %s", cur.c_str(), strerror(errno));
    if (next == std::string::npos) break;
    pos = next + 1;
  }
  return GOSSMX_OK;
}

// ---------------------------------------------------------------------------
// GOSSMX4 containers (RepackedMxfp4::open, cpu_repack.rs:231-280).

int layout_of(const RepackHeader& h) {
  for (int l = GOSSMX_LAYOUT_CANONICAL_V1; l <= GOSSMX_LAYOUT_GPU_TILED_V3; ++l)
    if (h.layout_version == (uint32_t)l && h.layout_identifier == layout_name(l)) return l;
  return 0;
}

bool payload_bytes_of(const RepackHeader& h, int layout, size_t& bytes) {
  const size_t e = h.shape[0], r = h.shape[1], b = h.shape[2];
  if (layout == GOSSMX_LAYOUT_GPU_TILED_V3) {
    // The tiled planes hold about 17 bytes per record plus tile padding.
    if (e == 0 || r == 0 || b == 0 || r > INT32_MAX || b > INT32_MAX || h.records > SIZE_MAX / 64) return false;
    size_t nib, scl;
    gossmx::tiled_image_bytes(e, r, b, &nib, &scl);
    bytes = nib + scl;
    return true;
  }
  if (h.records > SIZE_MAX / kRecordBytes) return false;
  bytes = h.records * kRecordBytes;
  return true;
}

struct Container {
  RepackHeader header;
  int layout = 0;
  size_t payload_offset = 0, payload_bytes = 0;
};

int read_container(const char* path, File& f, Container& c) {
  size_t size = 0;
  if (int s = open_read(path, f, size)) return s;
  char head[16];
  if (size < sizeof head) return err(GOSSMX_ERR_BAD_FILE, "invalid MXFP4 repack magic in %s", path);
  if (int s = read_exact(f.fd, head, sizeof head, 0, path)) return s;
  if (std::memcmp(head, kMagic, sizeof kMagic) != 0)
    return err(GOSSMX_ERR_BAD_FILE, "invalid MXFP4 repack magic in %s", path);
  uint64_t header_len = 0;
  for (int i = 0; i < 8; ++i) header_len |= (uint64_t)(uint8_t)head[8 + i] << (8 * i);
  if (header_len > kMaxHeaderBytes || header_len > size - sizeof head)
    return err(GOSSMX_ERR_BAD_FILE, "truncated MXFP4 repack header in %s", path);
  std::vector<char> text(header_len);
  if (int s = read_exact(f.fd, text.data(), header_len, sizeof head, path)) return s;
  Json j;
  JsonReader reader(text.data(), text.size());
  if (!reader.parse(j) || !c.header.parse(j)) return err(GOSSMX_ERR_BAD_FILE, "invalid repack header in %s", path);
  c.layout = layout_of(c.header);
  if (c.layout == 0)
    return err(GOSSMX_ERR_BAD_FILE, "unsupported MXFP4 repack layout %s version %u in %s",
               c.header.layout_identifier.c_str(), c.header.layout_version, path);
  const size_t* sh = c.header.shape;
  if (sh[1] != 0 && sh[0] > SIZE_MAX / sh[1]) return err(GOSSMX_ERR_BAD_FILE, "MXFP4 repack shape overflows");
  if (sh[2] != 0 && sh[0] * sh[1] > SIZE_MAX / sh[2]) return err(GOSSMX_ERR_BAD_FILE, "MXFP4 repack shape overflows");
  if (c.header.records != sh[0] * sh[1] * sh[2])
    return err(GOSSMX_ERR_BAD_FILE, "MXFP4 repack %s holds %zu records for shape [%zu, %zu, %zu]", path,
               c.header.records, sh[0], sh[1], sh[2]);
  c.payload_offset = sizeof head + (size_t)header_len;
  if (!payload_bytes_of(c.header, c.layout, c.payload_bytes) || c.payload_bytes > SIZE_MAX - c.payload_offset)
    return err(GOSSMX_ERR_BAD_FILE, "MXFP4 repack size overflows");
  if (size != c.payload_offset + c.payload_bytes)
    return err(GOSSMX_ERR_BAD_FILE, "MXFP4 repack %s has %zu bytes, expected %zu", path, size,
               c.payload_offset + c.payload_bytes);
  return GOSSMX_OK;
}

int load_container(gossmx_ctx* ctx, const char* path, const RepackHeader* expected, gossmx_weights** out) {
  File f;
  Container c;
  if (int s = read_container(path, f, c)) return s;
  if (expected && !(c.header == *expected))
    return err(GOSSMX_ERR_BAD_FILE, "stale MXFP4 repack metadata in %s", path);
  std::vector<uint8_t> payload(c.payload_bytes);
  if (int s = read_exact(f.fd, payload.data(), payload.size(), c.payload_offset, path)) return s;
  const size_t* sh = c.header.shape;
  if (c.layout == GOSSMX_LAYOUT_GPU_TILED_V3) {
    size_t nib = 0, scl = 0;
    gossmx::tiled_image_bytes(sh[0], sh[1], sh[2], &nib, &scl);
    return gossmx::tiled_image_create(ctx, sh[0], sh[1], sh[2], payload.data(), payload.data() + nib, out);
  }
  return gossmx_weights_upload(ctx, payload.data(), payload.size(), sh[0], sh[1], sh[2], c.layout, out);
}

// Writes the container to a temporary file beside `path`, syncs it, renames
// it over `path` and syncs the directory (cpu_repack.rs:190-204, 400-420).
int publish_container(const std::string& path, const RepackHeader& h, const uint8_t* a, size_t a_len,
                      const uint8_t* b, size_t b_len) {
  const std::string dir = parent_dir(path);
  const std::string tmp = dir + "/.weights.repack." + std::to_string((long)::getpid()) + ".tmp";
  const std::string text = h.serialize();
  uint8_t len[8];
  for (int i = 0; i < 8; ++i) len[i] = (uint8_t)((uint64_t)text.size() >> (8 * i));
  const int fd = ::open(tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
  if (fd < 0) return err(GOSSMX_ERR_BAD_FILE, "cannot create %s: %s", tmp.c_str(), strerror(errno));
  int s = write_all(fd, kMagic, sizeof kMagic, tmp.c_str());
  if (!s) s = write_all(fd, len, sizeof len, tmp.c_str());
  if (!s) s = write_all(fd, text.data(), text.size(), tmp.c_str());
  if (!s) s = write_all(fd, a, a_len, tmp.c_str());
  if (!s) s = write_all(fd, b, b_len, tmp.c_str());
  if (!s && ::fsync(fd) != 0) s = err(GOSSMX_ERR_BAD_FILE, "fsync of %s failed: %s", tmp.c_str(), strerror(errno));
  ::close(fd);
  if (!s && ::rename(tmp.c_str(), path.c_str()) != 0)
    s = err(GOSSMX_ERR_BAD_FILE, "cannot rename %s to %s: %s", tmp.c_str(), path.c_str(), strerror(errno));
  if (s) {
    ::unlink(tmp.c_str());
    return s;
  }
  return sync_directory(dir);
}

RepackHeader v3_header(const char* tensor_name, const size_t shape[3], const char* model_revision,
                       const char* const* hashes, size_t n_hashes) {
  RepackHeader h;
  h.layout_version = GOSSMX_LAYOUT_GPU_TILED_V3;
  h.layout_identifier = layout_name(GOSSMX_LAYOUT_GPU_TILED_V3);
  h.tensor_name = tensor_name;
  h.model_revision = model_revision;
  for (size_t i = 0; i < n_hashes; ++i) h.source_hashes.push_back(hashes[i]);
  for (int i = 0; i < 3; ++i) h.shape[i] = shape[i];
  h.records = shape[0] * shape[1] * shape[2];
  return h;
}

int save_v3(gossmx_ctx* ctx, const gossmx_weights* w, const std::string& path, const RepackHeader& h) {
  size_t nib = 0, scl = 0;
  gossmx::tiled_image_bytes(h.shape[0], h.shape[1], h.shape[2], &nib, &scl);
  std::vector<uint8_t> a(nib), b(scl);
  if (int s = gossmx::tiled_image_read(ctx, w, a.data(), b.data())) return s;
  return publish_container(path, h, a.data(), a.size(), b.data(), b.size());
}

// ---------------------------------------------------------------------------
// SafeTensors shards (parse_shard_header, cpu_tensor_store.rs:176-288).

size_t dtype_size(const std::string& d) {
  // DType::from_safetensors_str spellings.
  if (d == "BOOL" || d == "U8" || d == "I8" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
  if (d == "BF16" || d == "F16" || d == "I16" || d == "U16") return 2;
  if (d == "F32" || d == "I32" || d == "U32") return 4;
  if (d == "F64" || d == "I64" || d == "U64") return 8;
  return 0;
}

struct Tensor {
  std::string dtype;
  std::vector<size_t> shape;
  size_t start = 0, end = 0;  // absolute byte range in the shard
};

int shard_find(const char* path, const char* name, Tensor& t, bool& found) {
  found = false;
  File f;
  size_t size = 0;
  if (int s = open_read(path, f, size)) return s;
  uint8_t head[8];
  if (size < 8) return err(GOSSMX_ERR_BAD_FILE, "SafeTensors shard %s is too small", path);
  if (int s = read_exact(f.fd, head, 8, 0, path)) return s;
  uint64_t header_len = 0;
  for (int i = 0; i < 8; ++i) header_len |= (uint64_t)head[i] << (8 * i);
  if (header_len > kMaxHeaderBytes || header_len > size - 8)
    return err(GOSSMX_ERR_BAD_FILE, "SafeTensors header exceeds %s", path);
  const size_t data_start = 8 + (size_t)header_len;
  std::vector<char> text(header_len);
  if (int s = read_exact(f.fd, text.data(), header_len, 8, path)) return s;
  Json j;
  JsonReader reader(text.data(), text.size());
  if (!reader.parse(j) || j.kind != Json::kObject)
    return err(GOSSMX_ERR_BAD_FILE, "invalid SafeTensors header in %s", path);
  for (const auto& m : j.members) {
    if (m.first == "__metadata__") continue;
    const Json& v = m.second;
    const Json* dt = v.get("dtype");
    const Json* sh = v.get("shape");
    const Json* off = v.get("data_offsets");
    if (v.kind != Json::kObject || !dt || dt->kind != Json::kString || !sh || sh->kind != Json::kArray || !off ||
        off->kind != Json::kArray || off->items.size() != 2)
      return err(GOSSMX_ERR_BAD_FILE, "invalid metadata for tensor %s in %s", m.first.c_str(), path);
    const size_t es = dtype_size(dt->str);
    if (es == 0) return err(GOSSMX_ERR_BAD_FILE, "unsupported dtype %s for tensor %s", dt->str.c_str(), m.first.c_str());
    Tensor cur;
    cur.dtype = dt->str;
    size_t elements = 1;
    for (const Json& d : sh->items) {
      if (d.kind != Json::kNumber || !d.is_uint || d.uint > SIZE_MAX)
        return err(GOSSMX_ERR_BAD_FILE, "invalid metadata for tensor %s in %s", m.first.c_str(), path);
      if (d.uint != 0 && elements > SIZE_MAX / d.uint)
        return err(GOSSMX_ERR_BAD_FILE, "tensor %s shape overflows", m.first.c_str());
      elements *= (size_t)d.uint;
      cur.shape.push_back((size_t)d.uint);
    }
    for (const Json& o : off->items)
      if (o.kind != Json::kNumber || !o.is_uint || o.uint > SIZE_MAX - data_start)
        return err(GOSSMX_ERR_BAD_FILE, "tensor %s offset overflows", m.first.c_str());
    cur.start = data_start + (size_t)off->items[0].uint;
    cur.end = data_start + (size_t)off->items[1].uint;
    if (cur.start > cur.end || cur.end > size)
      return err(GOSSMX_ERR_BAD_FILE, "tensor %s has invalid byte range [%zu, %zu)", m.first.c_str(), cur.start,
                 cur.end);
    if (elements > SIZE_MAX / es) return err(GOSSMX_ERR_BAD_FILE, "tensor %s byte size overflows", m.first.c_str());
    if (elements * es != cur.end - cur.start)
      return err(GOSSMX_ERR_BAD_FILE, "tensor %s declares %zu bytes but stores %zu", m.first.c_str(), elements * es,
                 cur.end - cur.start);
    if (m.first == name) {
      if (found) return err(GOSSMX_ERR_BAD_FILE, "tensor %s occurs twice in %s", name, path);
      t = cur;
      found = true;
    }
  }
  return GOSSMX_OK;
}

// The tensor `name` in exactly one of the shards, as U8 bytes.
int shards_read_u8(const char* const* shards, size_t n, const char* name, Tensor& t, std::vector<uint8_t>& bytes) {
  int where = -1;
  for (size_t i = 0; i < n; ++i) {
    Tensor cur;
    bool found = false;
    if (int s = shard_find(shards[i], name, cur, found)) return s;
    if (!found) continue;
    if (where >= 0) return err(GOSSMX_ERR_BAD_FILE, "tensor %s occurs in more than one SafeTensors shard", name);
    where = (int)i;
    t = cur;
  }
  if (where < 0) return err(GOSSMX_ERR_BAD_FILE, "missing checkpoint tensor %s", name);
  if (t.dtype != "U8") return err(GOSSMX_ERR_BAD_FILE, "tensor %s has dtype %s, expected U8", name, t.dtype.c_str());
  File f;
  size_t size = 0;
  if (int s = open_read(shards[where], f, size)) return s;
  bytes.resize(t.end - t.start);
  return read_exact(f.fd, bytes.data(), bytes.size(), t.start, shards[where]);
}

// Canonical v1 records from the checkpoint tensors, with the source checks
// of open_or_create (cpu_repack.rs:155-174) and its record interleave
// (write_repack, cpu_repack.rs:412-425).
int from_safetensors(gossmx_ctx* ctx, const char* const* shards, size_t n_shards, const char* blocks_name,
                     const char* scales_name, gossmx_weights** out, size_t shape_out[3]) {
  Tensor bt, st;
  std::vector<uint8_t> blocks, scales;
  if (int s = shards_read_u8(shards, n_shards, blocks_name, bt, blocks)) return s;
  if (int s = shards_read_u8(shards, n_shards, scales_name, st, scales)) return s;
  if (bt.shape.size() != 4 || st.shape.size() != 3 || bt.shape[0] != st.shape[0] || bt.shape[1] != st.shape[1] ||
      bt.shape[2] != st.shape[2] || bt.shape[3] != 16)
    return err(GOSSMX_ERR_BAD_FILE, "invalid MXFP4 source shapes for %s", blocks_name);
  const size_t records = st.shape[0] * st.shape[1] * st.shape[2];
  if (blocks.size() != records * 16 || scales.size() != records)
    return err(GOSSMX_ERR_BAD_FILE, "invalid MXFP4 source byte counts for %s", blocks_name);
  std::vector<uint8_t> canonical(records * kRecordBytes);
  for (size_t r = 0; r < records; ++r) {
    canonical[r * kRecordBytes] = scales[r];
    std::memcpy(&canonical[r * kRecordBytes + 1], &blocks[r * 16], 16);
  }
  for (int i = 0; i < 3; ++i) shape_out[i] = st.shape[i];
  return gossmx_weights_upload(ctx, canonical.data(), canonical.size(), st.shape[0], st.shape[1], st.shape[2],
                               GOSSMX_LAYOUT_CANONICAL_V1, out);
}

// ---------------------------------------------------------------------------
// Lock file of open_or_create (acquire_lock, cpu_repack.rs:349-398).

bool lock_owner_is_gone(const std::string& path) {
  FILE* f = std::fopen(path.c_str(), "r");
  if (!f) return false;
  char line[128];
  long pid = -1;
  while (std::fgets(line, sizeof line, f))
    if (std::strncmp(line, "pid=", 4) == 0) {
      char* end = nullptr;
      const long v = std::strtol(line + 4, &end, 10);
      if (end != line + 4 && v > 0) pid = v;
      break;
    }
  std::fclose(f);
  if (pid <= 0) return false;
  struct stat st;
  return ::stat(("/proc/" + std::to_string(pid)).c_str(), &st) != 0;
}

int acquire_lock(const std::string& lock, const std::string& target, const RepackHeader& expected, bool& owned) {
  owned = false;
  const auto started = std::chrono::steady_clock::now();
  const auto limit = std::chrono::seconds(120);
  while (true) {
    const int fd = ::open(lock.c_str(), O_WRONLY | O_CREAT | O_EXCL | O_CLOEXEC, 0644);
    if (fd >= 0) {
      const std::string text = "pid=" + std::to_string((long)::getpid()) + "\n";
      int s = write_all(fd, text.data(), text.size(), lock.c_str());
      if (!s && ::fsync(fd) != 0) s = err(GOSSMX_ERR_BAD_FILE, "fsync of %s failed", lock.c_str());
      ::close(fd);
      if (s) {
        ::unlink(lock.c_str());
        return s;
      }
      owned = true;
      return GOSSMX_OK;
    }
    if (errno != EEXIST) return err(GOSSMX_ERR_BAD_FILE, "cannot create %s: %s", lock.c_str(), strerror(errno));
    if (lock_owner_is_gone(lock)) {
      ::unlink(lock.c_str());
      continue;
    }
    File f;
    Container c;
    if (read_container(target.c_str(), f, c) == GOSSMX_OK && c.header == expected) {
      // Another writer published; wait for it to release its lock.
      struct stat st;
      while (::stat(lock.c_str(), &st) == 0 && std::chrono::steady_clock::now() - started < limit)
        std::this_thread::sleep_for(std::chrono::milliseconds(25));
      continue;
    }
    if (std::chrono::steady_clock::now() - started >= limit)
      return err(GOSSMX_ERR_BAD_FILE, "timed out waiting for MXFP4 repack lock %s", lock.c_str());
    std::this_thread::sleep_for(std::chrono::milliseconds(50));
  }
}

}  // namespace

extern "C" {

int gossmx_repack_cache_key(const char* tensor_name, const size_t shape[3], int layout, const char* model_revision,
                            const char* const* source_hashes, size_t n_hashes, char key[65]) {
  const char* name = layout_name(layout);
  if (!tensor_name || !shape || !model_revision || (n_hashes && !source_hashes) || !key || !name)
    return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument or unknown layout");
  Sha256 d;
  const char prefix[] = "gpt-oss-rs-mxfp4-repack";
  d.update(prefix, sizeof prefix - 1);
  const uint32_t words[2] = {kFormatVersion, (uint32_t)layout};
  uint8_t le[8];
  for (int i = 0; i < 4; ++i) le[i] = (uint8_t)(words[0] >> (8 * i));
  d.update(le, 4);
  d.update(name, std::strlen(name));
  for (int i = 0; i < 4; ++i) le[i] = (uint8_t)(words[1] >> (8 * i));
  d.update(le, 4);
  d.update(model_revision, std::strlen(model_revision));
  for (size_t i = 0; i < n_hashes; ++i) {
    if (!source_hashes[i]) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null source hash");
    d.update(source_hashes[i], std::strlen(source_hashes[i]));
  }
  d.update(tensor_name, std::strlen(tensor_name));
  for (int k = 0; k < 3; ++k) {
    for (int i = 0; i < 8; ++i) le[i] = (uint8_t)((uint64_t)shape[k] >> (8 * i));
    d.update(le, 8);
  }
  d.hex(key);
  return GOSSMX_OK;
}

int gossmx_repack_inspect(const char* path, gossmx_repack_info* info, char* tensor_name, size_t cap) {
  if (!path || !info) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  File f;
  Container c;
  if (int s = read_container(path, f, c)) return s;
  info->format_version = c.header.format_version;
  info->layout_version = c.header.layout_version;
  info->experts = c.header.shape[0];
  info->rows = c.header.shape[1];
  info->blocks = c.header.shape[2];
  info->records = c.header.records;
  info->payload_offset = c.payload_offset;
  info->payload_bytes = c.payload_bytes;
  if (tensor_name && cap > 0) {
    const size_t n = std::min(cap - 1, c.header.tensor_name.size());
    std::memcpy(tensor_name, c.header.tensor_name.data(), n);
    tensor_name[n] = '\0';
  }
  return GOSSMX_OK;
}

int gossmx_weights_load_repack(gossmx_ctx* ctx, const char* path, gossmx_weights** out) {
  if (!ctx || !path || !out) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  return load_container(ctx, path, nullptr, out);
}

int gossmx_weights_save_repack(gossmx_ctx* ctx, const gossmx_weights* w, const char* path, const char* tensor_name,
                               const char* model_revision, const char* const* source_hashes, size_t n_hashes) {
  if (!ctx || !w || !path || !tensor_name || !model_revision || (n_hashes && !source_hashes))
    return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  for (size_t i = 0; i < n_hashes; ++i)
    if (!source_hashes[i]) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null source hash");
  size_t shape[3];
  if (int s = gossmx_weights_shape(w, &shape[0], &shape[1], &shape[2])) return s;
  return save_v3(ctx, w, path, v3_header(tensor_name, shape, model_revision, source_hashes, n_hashes));
}

int gossmx_safetensors_find(const char* path, const char* name, gossmx_tensor_info* info) {
  if (!path || !name || !info) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  Tensor t;
  bool found = false;
  if (int s = shard_find(path, name, t, found)) return s;
  if (!found) return err(GOSSMX_ERR_BAD_FILE, "missing checkpoint tensor %s in %s", name, path);
  if (t.shape.size() > sizeof info->shape / sizeof info->shape[0])
    return err(GOSSMX_ERR_UNSUPPORTED, "tensor %s has rank %zu", name, t.shape.size());
  std::memset(info, 0, sizeof *info);
  std::snprintf(info->dtype, sizeof info->dtype, "%s", t.dtype.c_str());
  info->rank = t.shape.size();
  for (size_t i = 0; i < t.shape.size(); ++i) info->shape[i] = t.shape[i];
  info->offset = t.start;
  info->bytes = t.end - t.start;
  return GOSSMX_OK;
}

int gossmx_weights_from_safetensors(gossmx_ctx* ctx, const char* const* shards, size_t n_shards,
                                    const char* blocks_name, const char* scales_name, gossmx_weights** out) {
  if (!ctx || !shards || n_shards == 0 || !blocks_name || !scales_name || !out)
    return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  for (size_t i = 0; i < n_shards; ++i)
    if (!shards[i]) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null shard path");
  size_t shape[3];
  return from_safetensors(ctx, shards, n_shards, blocks_name, scales_name, out, shape);
}

int gossmx_weights_open_or_create(gossmx_ctx* ctx, const char* cache_root, const char* model_revision,
                                  const char* const* source_hashes, size_t n_hashes, const char* const* shards,
                                  size_t n_shards, const char* blocks_name, const char* scales_name,
                                  gossmx_weights** out) {
  if (!ctx || !cache_root || !model_revision || (n_hashes && !source_hashes) || !shards || n_shards == 0 ||
      !blocks_name || !scales_name || !out)
    return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  for (size_t i = 0; i < n_hashes; ++i)
    if (!source_hashes[i]) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null source hash");
  for (size_t i = 0; i < n_shards; ++i)
    if (!shards[i]) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null shard path");
  // The key needs the source shape: the scales tensor's header.
  Tensor st;
  int where = -1;
  for (size_t i = 0; i < n_shards; ++i) {
    Tensor cur;
    bool found = false;
    if (int s = shard_find(shards[i], scales_name, cur, found)) return s;
    if (found) {
      if (where >= 0) return err(GOSSMX_ERR_BAD_FILE, "tensor %s occurs in more than one SafeTensors shard", scales_name);
      where = (int)i;
      st = cur;
    }
  }
  if (where < 0) return err(GOSSMX_ERR_BAD_FILE, "missing checkpoint tensor %s", scales_name);
  if (st.shape.size() != 3) return err(GOSSMX_ERR_BAD_FILE, "invalid MXFP4 source shapes for %s", blocks_name);
  const size_t shape[3] = {st.shape[0], st.shape[1], st.shape[2]};
  char key[65];
  if (int s = gossmx_repack_cache_key(blocks_name, shape, GOSSMX_LAYOUT_GPU_TILED_V3, model_revision, source_hashes,
                                      n_hashes, key))
    return s;
  const RepackHeader expected = v3_header(blocks_name, shape, model_revision, source_hashes, n_hashes);
  const std::string dir = std::string(cache_root) + "/mxfp4/" + key;
  const std::string target = dir + "/weights.repack";
  if (load_container(ctx, target.c_str(), &expected, out) == GOSSMX_OK) {
    gossmx::count_repack_cache(true);
    return GOSSMX_OK;
  }
  if (int s = make_dirs(dir)) return s;
  const std::string lock = dir + "/repack.lock";
  bool owned = false;
  if (int s = acquire_lock(lock, target, expected, owned)) return s;
  int s = load_container(ctx, target.c_str(), &expected, out);
  gossmx::count_repack_cache(s == GOSSMX_OK);
  if (s != GOSSMX_OK) {
    size_t got[3];
    s = from_safetensors(ctx, shards, n_shards, blocks_name, scales_name, out, got);
    if (s == GOSSMX_OK) {
      s = save_v3(ctx, *out, target, expected);
      if (s != GOSSMX_OK) {
        gossmx_weights_destroy(*out);
        *out = nullptr;
      }
    }
  }
  if (owned) ::unlink(lock.c_str());
  return s;
}

}  // extern "C"
