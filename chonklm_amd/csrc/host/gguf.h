// GGUF v2/v3 container: byte sources (single file, shard manifest, memory),
// header parser and writer.
//
// Parser semantics follow src/lib/gguf.ts:42-101 of the reference:
//   * magic "GGUF" (0x46554747 little-endian), version, u64 tensor/kv counts;
//   * metadata value types 0..12 with arrays;
//   * tensor infos (name, dims, type, offset) with byte length computed by
//     tensor_byte_length;
//   * data offset = header end rounded up to 32 bytes (general.alignment is
//     not consulted, as in the reference);
//   * the header must parse within the first 64 MiB (gguf.ts:43-55).
// Shard manifests follow scripts/shard-gguf.mjs:152-160 and the logical range
// semantics of fetchShardedRange (src/lib/cache.ts:422-467).
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace chonk {

// ---- byte sources --------------------------------------------------------------

class ByteSource {
 public:
  virtual ~ByteSource() = default;
  virtual uint64_t size() const = 0;
  // Reads [offset, offset+length) into dst; throws std::runtime_error on a
  // range outside the source or an I/O error.
  virtual void read(uint64_t offset, uint64_t length, void* dst) const = 0;
};

struct ShardEntry {
  int64_t index = 0;
  std::string name;
  uint64_t offset = 0;
  uint64_t size = 0;
};

struct ShardManifest {
  int64_t version = 0;
  std::string quant;
  uint64_t total_size = 0;
  uint64_t shard_size = 0;
  int64_t shard_count = 0;
  std::vector<ShardEntry> shards;
};

// Parses manifest.json text (the sharder's schema). Throws on malformed input.
ShardManifest parse_shard_manifest(const std::string& json_text);
std::string shard_manifest_to_json(const ShardManifest& m);

// Opens a .gguf file, or a directory holding manifest.json + NNNN.bin shards.
std::unique_ptr<ByteSource> open_byte_source(const std::string& path);
// Wraps a caller buffer (copied).
std::unique_ptr<ByteSource> memory_byte_source(const void* data, uint64_t size);

// Splits a GGUF file into <out_dir>/NNNN.bin shards of at most shard_size
// bytes plus manifest.json (scripts/shard-gguf.mjs:102-167).
ShardManifest write_shards(const std::string& gguf_path, const std::string& out_dir, uint64_t shard_size,
                           const std::string& quant);

// ---- metadata ------------------------------------------------------------------

enum GgufValueType : uint32_t {
  GV_U8 = 0, GV_I8 = 1, GV_U16 = 2, GV_I16 = 3, GV_U32 = 4, GV_I32 = 5, GV_F32 = 6,
  GV_BOOL = 7, GV_STRING = 8, GV_ARRAY = 9, GV_U64 = 10, GV_I64 = 11, GV_F64 = 12,
};

struct GgufValue {
  GgufValueType type = GV_U32;
  // Numeric payload as double (integers up to 2^53 are exact), also the raw
  // 64-bit integer for the integer types.
  double number = 0;
  int64_t i64 = 0;
  uint64_t u64 = 0;
  bool boolean = false;
  std::string str;
  std::vector<GgufValue> array;

  bool is_number() const {
    return type != GV_STRING && type != GV_ARRAY && type != GV_BOOL;
  }
};

struct GgufTensorInfo {
  std::string name;
  std::vector<uint64_t> shape;  // GGUF order: shape[0] is the row length
  uint32_t type = 0;
  uint64_t offset = 0;          // relative to data_offset
  uint64_t n_elements = 0;
  uint64_t n_bytes = 0;
};

struct GgufFile {
  uint32_t version = 0;
  uint64_t tensor_count = 0;
  uint64_t kv_count = 0;
  std::map<std::string, GgufValue> kv;
  std::vector<GgufTensorInfo> tensors;
  std::map<std::string, size_t> tensor_index;
  uint64_t data_offset = 0;

  const GgufTensorInfo* find(const std::string& name) const {
    auto it = tensor_index.find(name);
    return it == tensor_index.end() ? nullptr : &tensors[it->second];
  }
  const GgufValue* value(const std::string& key) const {
    auto it = kv.find(key);
    return it == kv.end() ? nullptr : &it->second;
  }
};

// Parses a header from bytes already in memory; throws std::runtime_error
// ("invalid GGUF magic: 0x...", "unsupported GGUF metadata value type N", ...).
GgufFile parse_gguf(const uint8_t* bytes, uint64_t size);
// Reads the header from a source with the 4 MiB -> 64 MiB doubling window.
GgufFile read_gguf_header(const ByteSource& src, const std::string& label);

// ---- writer --------------------------------------------------------------------

class GgufWriter {
 public:
  void set_string(const std::string& key, const std::string& v);
  void set_u32(const std::string& key, uint32_t v);
  void set_i32(const std::string& key, int32_t v);
  void set_f32(const std::string& key, float v);
  void set_bool(const std::string& key, bool v);
  void set_u32_array(const std::string& key, const std::vector<uint32_t>& v);
  // Adds a tensor; shape in GGUF order (row length first). data must hold
  // tensor_byte_length(type, prod(shape)) bytes and is copied.
  void add_tensor(const std::string& name, const std::vector<uint64_t>& shape, uint32_t type,
                  std::vector<uint8_t> data);
  // Writes version-3 GGUF with 32-byte aligned tensor data.
  void write(const std::string& path) const;

 private:
  struct KV {
    std::string key;
    std::vector<uint8_t> encoded;  // type tag + payload
  };
  struct Tensor {
    std::string name;
    std::vector<uint64_t> shape;
    uint32_t type;
    std::vector<uint8_t> data;
  };
  std::vector<KV> kvs_;
  std::vector<Tensor> tensors_;
};

}  // namespace chonk
