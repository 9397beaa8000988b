// GGUF container I/O; see gguf.h for the reference semantics it follows.
#include "gguf.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <sstream>
#include <stdexcept>

#include "ggml_types.h"

namespace chonk {

// ---- byte sources --------------------------------------------------------------

namespace {

std::string hex32(uint32_t v) {
  char buf[16];
  std::snprintf(buf, sizeof buf, "%x", v);
  return buf;
}

void pread_all(int fd, uint64_t offset, uint64_t length, void* dst, const std::string& label) {
  uint8_t* p = static_cast<uint8_t*>(dst);
  while (length > 0) {
    const size_t chunk = (size_t)std::min<uint64_t>(length, 1ull << 30);
    const ssize_t n = ::pread(fd, p, chunk, (off_t)offset);
    if (n < 0) {
      if (errno == EINTR) continue;
      throw std::runtime_error("read failed for " + label + ": " + std::strerror(errno));
    }
    if (n == 0) throw std::runtime_error("unexpected end of file in " + label);
    p += n;
    offset += (uint64_t)n;
    length -= (uint64_t)n;
  }
}

class FileSource : public ByteSource {
 public:
  explicit FileSource(const std::string& path) : path_(path) {
    fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd_ < 0) throw std::runtime_error("cannot open " + path + ": " + std::strerror(errno));
    struct stat st;
    if (::fstat(fd_, &st) != 0) {
      ::close(fd_);
      throw std::runtime_error("cannot stat " + path);
    }
    size_ = (uint64_t)st.st_size;
  }
  ~FileSource() override { ::close(fd_); }
  uint64_t size() const override { return size_; }
  void read(uint64_t offset, uint64_t length, void* dst) const override {
    if (offset + length > size_ || offset + length < offset) {
      throw std::runtime_error("range out of bounds for " + path_ + ": offset=" + std::to_string(offset) +
                               " length=" + std::to_string(length) + " totalSize=" + std::to_string(size_));
    }
    pread_all(fd_, offset, length, dst, path_);
  }

 private:
  std::string path_;
  int fd_ = -1;
  uint64_t size_ = 0;
};

class MemorySource : public ByteSource {
 public:
  MemorySource(const void* data, uint64_t size)
      : bytes_(static_cast<const uint8_t*>(data), static_cast<const uint8_t*>(data) + size) {}
  uint64_t size() const override { return bytes_.size(); }
  void read(uint64_t offset, uint64_t length, void* dst) const override {
    if (offset + length > bytes_.size() || offset + length < offset) {
      throw std::runtime_error("range out of bounds for memory source: offset=" + std::to_string(offset) +
                               " length=" + std::to_string(length) +
                               " totalSize=" + std::to_string(bytes_.size()));
    }
    if (length) std::memcpy(dst, bytes_.data() + offset, (size_t)length);
  }

 private:
  std::vector<uint8_t> bytes_;
};

// A logical byte range over contiguous shards (src/lib/cache.ts:422-467).
class ShardSource : public ByteSource {
 public:
  ShardSource(const std::string& dir, ShardManifest m) : dir_(dir), m_(std::move(m)) {
    uint64_t expect = 0;
    for (const auto& s : m_.shards) {
      if (s.offset != expect) throw std::runtime_error("shard manifest for " + dir_ + " is not contiguous");
      expect += s.size;
      const std::string path = dir_ + "/" + s.name;
      struct stat st;
      if (::stat(path.c_str(), &st) != 0) throw std::runtime_error("missing shard " + path);
      // cache.ts:568-573 rejects a shard whose byte size differs from the manifest,
      // with this wording
      if ((uint64_t)st.st_size != s.size) {
        throw std::runtime_error("shard " + path + ": expected " + std::to_string(s.size) + " bytes, got " +
                                 std::to_string((uint64_t)st.st_size));
      }
    }
    if (expect != m_.total_size) throw std::runtime_error("shard manifest totalSize mismatch for " + dir_);
  }
  uint64_t size() const override { return m_.total_size; }
  void read(uint64_t offset, uint64_t length, void* dst) const override {
    if (offset + length > m_.total_size || offset + length < offset) {
      throw std::runtime_error("range out of bounds for " + dir_ + ": offset=" + std::to_string(offset) +
                               " length=" + std::to_string(length) + " totalSize=" + std::to_string(m_.total_size));
    }
    const uint64_t end = offset + length;
    uint8_t* out = static_cast<uint8_t*>(dst);
    for (const auto& s : m_.shards) {
      const uint64_t s_end = s.offset + s.size;
      if (s_end <= offset) continue;
      if (s.offset >= end) break;
      const uint64_t lo = std::max(offset, s.offset);
      const uint64_t hi = std::min(end, s_end);
      const std::string path = dir_ + "/" + s.name;
      int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
      if (fd < 0) throw std::runtime_error("cannot open shard " + path);
      try {
        pread_all(fd, lo - s.offset, hi - lo, out + (lo - offset), path);
      } catch (...) {
        ::close(fd);
        throw;
      }
      ::close(fd);
    }
  }

 private:
  std::string dir_;
  ShardManifest m_;
};

// ---- a small JSON reader for the manifest schema --------------------------------

struct Json {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  double num = 0;
  bool b = false;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
  const Json* get(const std::string& k) const {
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

class JsonParser {
 public:
  explicit JsonParser(const std::string& s) : s_(s) {}
  Json parse() {
    Json v = value();
    ws();
    if (i_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void fail(const char* what) {
    throw std::runtime_error(std::string("malformed shard manifest JSON: ") + what + " at byte " +
                             std::to_string(i_));
  }
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
  }
  Json value() {
    ws();
    if (i_ >= s_.size()) fail("unexpected end");
    const char c = s_[i_];
    Json v;
    if (c == '{') {
      v.kind = Json::OBJ;
      ++i_;
      ws();
      if (i_ < s_.size() && s_[i_] == '}') {
        ++i_;
        return v;
      }
      while (true) {
        ws();
        if (i_ >= s_.size() || s_[i_] != '"') fail("expected key");
        std::string k = string();
        ws();
        if (i_ >= s_.size() || s_[i_] != ':') fail("expected ':'");
        ++i_;
        v.obj.emplace_back(std::move(k), value());
        ws();
        if (i_ < s_.size() && s_[i_] == ',') {
          ++i_;
          continue;
        }
        if (i_ < s_.size() && s_[i_] == '}') {
          ++i_;
          return v;
        }
        fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind = Json::ARR;
      ++i_;
      ws();
      if (i_ < s_.size() && s_[i_] == ']') {
        ++i_;
        return v;
      }
      while (true) {
        v.arr.push_back(value());
        ws();
        if (i_ < s_.size() && s_[i_] == ',') {
          ++i_;
          continue;
        }
        if (i_ < s_.size() && s_[i_] == ']') {
          ++i_;
          return v;
        }
        fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Json::STR;
      v.str = string();
      return v;
    }
    if (s_.compare(i_, 4, "true") == 0) {
      v.kind = Json::BOOL;
      v.b = true;
      i_ += 4;
      return v;
    }
    if (s_.compare(i_, 5, "false") == 0) {
      v.kind = Json::BOOL;
      i_ += 5;
      return v;
    }
    if (s_.compare(i_, 4, "null") == 0) {
      i_ += 4;
      return v;
    }
    size_t end = i_;
    while (end < s_.size() && std::strchr("+-0123456789.eE", s_[end])) ++end;
    if (end == i_) fail("unexpected character");
    v.kind = Json::NUM;
    v.num = std::strtod(s_.substr(i_, end - i_).c_str(), nullptr);
    i_ = end;
    return v;
  }
  std::string string() {
    ++i_;  // opening quote
    std::string out;
    while (i_ < s_.size() && s_[i_] != '"') {
      if (s_[i_] == '\\') {
        ++i_;
        if (i_ >= s_.size()) fail("bad escape");
        const char e = s_[i_];
        if (e == 'n') out += '\n';
        else if (e == 't') out += '\t';
        else if (e == 'r') out += '\r';
        else if (e == 'b') out += '\b';
        else if (e == 'f') out += '\f';
        else if (e == 'u') {
          if (i_ + 4 >= s_.size()) fail("bad \\u escape");
          const unsigned code = (unsigned)std::strtoul(s_.substr(i_ + 1, 4).c_str(), nullptr, 16);
          if (code < 0x80) out += (char)code;
          else fail("non-ASCII \\u escape unsupported");
          i_ += 4;
        } else out += e;
        ++i_;
      } else {
        out += s_[i_++];
      }
    }
    if (i_ >= s_.size()) fail("unterminated string");
    ++i_;
    return out;
  }
  const std::string& s_;
  size_t i_ = 0;
};

uint64_t json_u64(const Json& o, const char* key, bool required = true) {
  const Json* v = o.get(key);
  if (!v || v->kind != Json::NUM || v->num < 0) {
    if (!required) return 0;
    throw std::runtime_error(std::string("shard manifest field ") + key + " missing or not a non-negative number");
  }
  return (uint64_t)v->num;
}

std::string read_text_file(const std::string& path) {
  FileSource f(path);
  std::string s((size_t)f.size(), '\0');
  if (!s.empty()) f.read(0, f.size(), &s[0]);
  return s;
}

}  // namespace

ShardManifest parse_shard_manifest(const std::string& json_text) {
  Json root = JsonParser(json_text).parse();
  if (root.kind != Json::OBJ) throw std::runtime_error("shard manifest is not a JSON object");
  ShardManifest m;
  m.version = (int64_t)json_u64(root, "version", false);
  if (const Json* q = root.get("quant"); q && q->kind == Json::STR) m.quant = q->str;
  m.total_size = json_u64(root, "totalSize");
  m.shard_size = json_u64(root, "shardSize", false);
  const Json* shards = root.get("shards");
  if (!shards || shards->kind != Json::ARR) throw std::runtime_error("shard manifest has no shards array");
  for (const Json& s : shards->arr) {
    if (s.kind != Json::OBJ) throw std::runtime_error("shard manifest entry is not an object");
    ShardEntry e;
    e.index = (int64_t)json_u64(s, "index", false);
    const Json* name = s.get("name");
    if (!name || name->kind != Json::STR) throw std::runtime_error("shard manifest entry without name");
    if (name->str.find('/') != std::string::npos || name->str == "..") {
      throw std::runtime_error("shard name must be a plain file name: " + name->str);
    }
    e.name = name->str;
    e.offset = json_u64(s, "offset");
    e.size = json_u64(s, "size");
    m.shards.push_back(std::move(e));
  }
  m.shard_count = root.get("shardCount") ? (int64_t)json_u64(root, "shardCount") : (int64_t)m.shards.size();
  if (m.shard_count != (int64_t)m.shards.size()) throw std::runtime_error("shard manifest shardCount mismatch");
  return m;
}

std::string shard_manifest_to_json(const ShardManifest& m) {
  std::ostringstream o;
  o << "{\n  \"version\": " << m.version << ",\n  \"quant\": \"" << m.quant << "\",\n  \"totalSize\": "
    << m.total_size << ",\n  \"shardSize\": " << m.shard_size << ",\n  \"shardCount\": " << m.shards.size()
    << ",\n  \"shards\": [";
  for (size_t i = 0; i < m.shards.size(); ++i) {
    const auto& s = m.shards[i];
    o << (i ? ",\n" : "\n") << "    {\n      \"index\": " << s.index << ",\n      \"name\": \"" << s.name
      << "\",\n      \"offset\": " << s.offset << ",\n      \"size\": " << s.size << "\n    }";
  }
  o << "\n  ]\n}\n";
  return o.str();
}

std::unique_ptr<ByteSource> open_byte_source(const std::string& path) {
  struct stat st;
  if (::stat(path.c_str(), &st) != 0) throw std::runtime_error("cannot open " + path + ": " + std::strerror(errno));
  if (S_ISDIR(st.st_mode)) {
    const std::string mpath = path + "/manifest.json";
    return std::unique_ptr<ByteSource>(new ShardSource(path, parse_shard_manifest(read_text_file(mpath))));
  }
  return std::unique_ptr<ByteSource>(new FileSource(path));
}

std::unique_ptr<ByteSource> memory_byte_source(const void* data, uint64_t size) {
  return std::unique_ptr<ByteSource>(new MemorySource(data, size));
}

ShardManifest write_shards(const std::string& gguf_path, const std::string& out_dir, uint64_t shard_size,
                           const std::string& quant) {
  if (shard_size == 0) throw std::runtime_error("shard size must be positive");
  FileSource src(gguf_path);
  ::mkdir(out_dir.c_str(), 0755);
  ShardManifest m;
  m.version = 1;
  m.quant = quant;
  m.total_size = src.size();
  m.shard_size = shard_size;
  std::vector<uint8_t> buf;
  uint64_t off = 0;
  int64_t idx = 0;
  while (off < src.size() || (src.size() == 0 && idx == 0)) {
    const uint64_t n = std::min<uint64_t>(shard_size, src.size() - off);
    buf.resize((size_t)n);
    if (n) src.read(off, n, buf.data());
    char name[32];
    std::snprintf(name, sizeof name, "%04lld.bin", (long long)idx);
    const std::string path = out_dir + "/" + name;
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) throw std::runtime_error("cannot write " + path);
    const size_t w = n ? std::fwrite(buf.data(), 1, (size_t)n, f) : 0;
    std::fclose(f);
    if (w != n) throw std::runtime_error("short write to " + path);
    m.shards.push_back({idx, name, off, n});
    off += n;
    ++idx;
    if (n == 0) break;
  }
  m.shard_count = (int64_t)m.shards.size();
  const std::string mpath = out_dir + "/manifest.json";
  FILE* f = std::fopen(mpath.c_str(), "wb");
  if (!f) throw std::runtime_error("cannot write " + mpath);
  const std::string js = shard_manifest_to_json(m);
  std::fwrite(js.data(), 1, js.size(), f);
  std::fclose(f);
  return m;
}

// ---- parser --------------------------------------------------------------------

namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;  // "GGUF"

class Reader {
 public:
  Reader(const uint8_t* p, uint64_t n) : p_(p), n_(n) {}
  uint64_t offset() const { return off_; }
  void need(uint64_t k) {
    if (off_ + k > n_ || off_ + k < off_) throw std::runtime_error("GGUF header truncated");
  }
  template <typename T>
  T get() {
    need(sizeof(T));
    T v;
    std::memcpy(&v, p_ + off_, sizeof(T));
    off_ += sizeof(T);
    return v;
  }
  std::string str() {
    const uint64_t len = get<uint64_t>();
    need(len);
    std::string s(reinterpret_cast<const char*>(p_ + off_), (size_t)len);
    off_ += len;
    return s;
  }
  GgufValue value(uint32_t type, int depth = 0) {
    GgufValue v;
    v.type = (GgufValueType)type;
    switch (type) {
      case GV_U8: v.u64 = get<uint8_t>(); v.i64 = (int64_t)v.u64; v.number = (double)v.u64; break;
      case GV_I8: v.i64 = get<int8_t>(); v.number = (double)v.i64; break;
      case GV_U16: v.u64 = get<uint16_t>(); v.i64 = (int64_t)v.u64; v.number = (double)v.u64; break;
      case GV_I16: v.i64 = get<int16_t>(); v.number = (double)v.i64; break;
      case GV_U32: v.u64 = get<uint32_t>(); v.i64 = (int64_t)v.u64; v.number = (double)v.u64; break;
      case GV_I32: v.i64 = get<int32_t>(); v.number = (double)v.i64; break;
      case GV_F32: v.number = (double)get<float>(); break;
      case GV_BOOL: v.boolean = get<uint8_t>() != 0; v.number = v.boolean; break;
      case GV_STRING: v.str = str(); break;
      case GV_ARRAY: {
        if (depth > 4) throw std::runtime_error("GGUF metadata arrays nested too deeply");
        const uint32_t item = get<uint32_t>();
        const uint64_t len = get<uint64_t>();
        if (len > n_) throw std::runtime_error("GGUF header truncated");
        v.array.reserve((size_t)std::min<uint64_t>(len, 1u << 20));
        for (uint64_t i = 0; i < len; ++i) v.array.push_back(value(item, depth + 1));
        break;
      }
      case GV_U64: v.u64 = get<uint64_t>(); v.i64 = (int64_t)v.u64; v.number = (double)v.u64; break;
      case GV_I64: v.i64 = get<int64_t>(); v.number = (double)v.i64; break;
      case GV_F64: v.number = get<double>(); break;
      default: throw std::runtime_error("unsupported GGUF metadata value type " + std::to_string(type));
    }
    return v;
  }

 private:
  const uint8_t* p_;
  uint64_t n_;
  uint64_t off_ = 0;
};

}  // namespace

GgufFile parse_gguf(const uint8_t* bytes, uint64_t size) {
  Reader r(bytes, size);
  const uint32_t magic = r.get<uint32_t>();
  if (magic != kGgufMagic) throw std::runtime_error("invalid GGUF magic: 0x" + hex32(magic));
  GgufFile g;
  g.version = r.get<uint32_t>();
  g.tensor_count = r.get<uint64_t>();
  g.kv_count = r.get<uint64_t>();
  if (g.kv_count > size || g.tensor_count > size) throw std::runtime_error("GGUF header truncated");
  for (uint64_t i = 0; i < g.kv_count; ++i) {
    std::string key = r.str();
    const uint32_t type = r.get<uint32_t>();
    g.kv[key] = r.value(type);
  }
  for (uint64_t i = 0; i < g.tensor_count; ++i) {
    GgufTensorInfo t;
    t.name = r.str();
    const uint32_t nd = r.get<uint32_t>();
    if (nd > 8) throw std::runtime_error("GGUF tensor " + t.name + " has too many dimensions");
    t.n_elements = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      t.shape.push_back(r.get<uint64_t>());
      t.n_elements *= t.shape.back();
    }
    t.type = r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    t.n_bytes = tensor_byte_length(t.type, t.n_elements);
    g.tensor_index[t.name] = g.tensors.size();
    g.tensors.push_back(std::move(t));
  }
  g.data_offset = (r.offset() + 31) / 32 * 32;
  return g;
}

GgufFile read_gguf_header(const ByteSource& src, const std::string& label) {
  uint64_t window = 4ull << 20;
  std::string last_error;
  std::vector<uint8_t> buf;
  while (window <= (64ull << 20)) {
    const uint64_t n = std::min<uint64_t>(window, src.size());
    buf.resize((size_t)n);
    if (n) src.read(0, n, buf.data());
    try {
      GgufFile g = parse_gguf(buf.data(), n);
      if (g.data_offset <= n) return g;
      last_error = "GGUF header extends past " + std::to_string(window) + " bytes";
    } catch (const std::exception& e) {
      last_error = e.what();
    }
    if (n == src.size()) break;  // nothing more to read
    window *= 2;
  }
  throw std::runtime_error("could not parse GGUF header for " + label + ": Error: " + last_error);
}

// ---- writer --------------------------------------------------------------------

namespace {
template <typename T>
void put(std::vector<uint8_t>& out, T v) {
  const uint8_t* p = reinterpret_cast<const uint8_t*>(&v);
  out.insert(out.end(), p, p + sizeof(T));
}
void put_str(std::vector<uint8_t>& out, const std::string& s) {
  put<uint64_t>(out, s.size());
  out.insert(out.end(), s.begin(), s.end());
}
}  // namespace

void GgufWriter::set_string(const std::string& key, const std::string& v) {
  KV kv{key, {}};
  put<uint32_t>(kv.encoded, GV_STRING);
  put_str(kv.encoded, v);
  kvs_.push_back(std::move(kv));
}
void GgufWriter::set_u32(const std::string& key, uint32_t v) {
  KV kv{key, {}};
  put<uint32_t>(kv.encoded, GV_U32);
  put<uint32_t>(kv.encoded, v);
  kvs_.push_back(std::move(kv));
}
void GgufWriter::set_i32(const std::string& key, int32_t v) {
  KV kv{key, {}};
  put<uint32_t>(kv.encoded, GV_I32);
  put<int32_t>(kv.encoded, v);
  kvs_.push_back(std::move(kv));
}
void GgufWriter::set_f32(const std::string& key, float v) {
  KV kv{key, {}};
  put<uint32_t>(kv.encoded, GV_F32);
  put<float>(kv.encoded, v);
  kvs_.push_back(std::move(kv));
}
void GgufWriter::set_bool(const std::string& key, bool v) {
  KV kv{key, {}};
  put<uint32_t>(kv.encoded, GV_BOOL);
  put<uint8_t>(kv.encoded, v ? 1 : 0);
  kvs_.push_back(std::move(kv));
}
void GgufWriter::set_u32_array(const std::string& key, const std::vector<uint32_t>& v) {
  KV kv{key, {}};
  put<uint32_t>(kv.encoded, GV_ARRAY);
  put<uint32_t>(kv.encoded, GV_U32);
  put<uint64_t>(kv.encoded, v.size());
  for (uint32_t x : v) put<uint32_t>(kv.encoded, x);
  kvs_.push_back(std::move(kv));
}

void GgufWriter::add_tensor(const std::string& name, const std::vector<uint64_t>& shape, uint32_t type,
                            std::vector<uint8_t> data) {
  uint64_t n = 1;
  for (uint64_t d : shape) n *= d;
  if (data.size() != tensor_byte_length(type, n)) {
    throw std::runtime_error("GGUF writer: tensor " + name + " has " + std::to_string(data.size()) +
                             " bytes, expected " + std::to_string(tensor_byte_length(type, n)));
  }
  tensors_.push_back({name, shape, type, std::move(data)});
}

void GgufWriter::write(const std::string& path) const {
  std::vector<uint8_t> head;
  put<uint32_t>(head, kGgufMagic);
  put<uint32_t>(head, 3);
  put<uint64_t>(head, tensors_.size());
  put<uint64_t>(head, kvs_.size());
  for (const auto& kv : kvs_) {
    put_str(head, kv.key);
    head.insert(head.end(), kv.encoded.begin(), kv.encoded.end());
  }
  uint64_t off = 0;
  std::vector<uint64_t> offsets;
  for (const auto& t : tensors_) {
    put_str(head, t.name);
    put<uint32_t>(head, (uint32_t)t.shape.size());
    for (uint64_t d : t.shape) put<uint64_t>(head, d);
    put<uint32_t>(head, t.type);
    put<uint64_t>(head, off);
    offsets.push_back(off);
    off += (t.data.size() + 31) / 32 * 32;
  }
  head.resize((head.size() + 31) / 32 * 32, 0);
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f) throw std::runtime_error("cannot write " + path);
  bool ok = std::fwrite(head.data(), 1, head.size(), f) == head.size();
  static const uint8_t zeros[32] = {0};
  for (const auto& t : tensors_) {
    ok = ok && std::fwrite(t.data.data(), 1, t.data.size(), f) == t.data.size();
    const size_t pad = (32 - t.data.size() % 32) % 32;
    ok = ok && std::fwrite(zeros, 1, pad, f) == pad;
  }
  ok = (std::fclose(f) == 0) && ok;
  if (!ok) throw std::runtime_error("short write to " + path);
}

}  // namespace chonk
