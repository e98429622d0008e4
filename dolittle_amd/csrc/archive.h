// Checkpoint archives on the host: a bounded JSON reader, the safetensors
// header decoder and verified archive opening
// (src/tensors/formats/safetensors.h:101-117, safetensors.cpp), and the
// Qwen3 config and parameter binding (src/models/qwen3/checkpoint.h:104-123,
// checkpoint.cpp).  Pure host code: nothing here touches the GPU.  Errors map
// to the reference's exception classes: malformed or unsupported data ->
// DL_INVALID_ARGUMENT, limits and overflow -> DL_LENGTH_ERROR, I/O and digest
// mismatch -> DL_RUNTIME_ERROR.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

#include "../../include/dolittle_hip.h"

namespace dl::json {

// A parsed JSON value; objects keep their members in document order.
struct Value {
  enum Kind : uint8_t { kNull, kBool, kUnsigned, kSigned, kFloat, kString, kArray, kObject };
  Kind kind = kNull;
  bool boolean = false;
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0.0;
  std::string text;
  std::vector<Value> items;
  std::vector<std::pair<std::string, Value>> members;

  const Value* find(std::string_view key) const;
  bool is_integer() const { return kind == kUnsigned || kind == kSigned; }
  bool is_number() const { return is_integer() || kind == kFloat; }
  double number() const;
};

struct Document {
  Value value;
  uint64_t metadata_bytes;  // input bytes plus the charged node/string accounting
};

// Bounded parse (json_metadata.h:131-158): input above `limit` or accounting
// above what remains is DL_LENGTH_ERROR; duplicate keys at any depth,
// malformed text, nonfinite numbers and a non-object root are
// DL_INVALID_ARGUMENT; nesting is capped at 64 containers.
Document parse(const char* text, uint64_t bytes, uint64_t limit);
// A non-negative integer (json_metadata.h:160-173).
uint64_t unsigned_integer(const Value& v);
// Adds `amount` to `used` within `limit` (DL_LENGTH_ERROR beyond it).
void charge(uint64_t& used, uint64_t amount, uint64_t limit);

}  // namespace dl::json

namespace dl::archive {

constexpr int kU32 = 3;  // dl_dtype extension for U32 tensors (safetensors "U32")

struct Limits {
  uint64_t max_header_bytes, max_metadata_bytes, max_tensor_count;
};

// Byte size of a contiguous tensor; DL_LENGTH_ERROR when it overflows.
uint64_t required_bytes(int dtype, const std::vector<uint64_t>& shape);

struct Tensor {
  std::string name;
  int dtype = 0;
  std::vector<uint64_t> shape;
  uint64_t data_offset = 0, byte_count = 0;
  const uint8_t* payload = nullptr;  // null for a parsed header without a file
  std::string shard;
};

struct Tensors {
  std::vector<Tensor> ranges;  // sorted by name, as the reference's ordered JSON objects iterate
  uint64_t metadata_bytes = 0;
};

// safetensors::parse_header (safetensors.cpp decode_header).
Tensors decode_header(const char* json, uint64_t bytes, uint64_t data_bytes, Limits limits);

// SHA-256 (FIPS 180-4) of a byte range as 64 lowercase hex characters.
std::string sha256_hex(const uint8_t* data, uint64_t bytes);

struct Mapping;

}  // namespace dl::archive

// An opened archive or a decoded header (catalog without payloads).
struct dl_archive {
  std::string repository, revision, digest;
  std::vector<dl::archive::Tensor> catalog;
  std::map<std::string, size_t, std::less<>> by_name;
  std::map<std::string, std::unique_ptr<dl::archive::Mapping>, std::less<>> artifacts;
  const dl::archive::Tensor& tensor(std::string_view name) const;
  std::pair<const uint8_t*, uint64_t> artifact(std::string_view path) const;
  ~dl_archive();
};

namespace dl::qwen3 {

struct Settings {
  dl_qwen3_config config{};
  uint64_t context_limit = 0;
  int weight_dtype = 0;
};

// parse_config (checkpoint.cpp:197-287) into this backend's config struct;
// dimensions above 32 bits are DL_LENGTH_ERROR here.
Settings parse_config(const char* json, uint64_t bytes, int actual_weight_dtype, uint64_t max_metadata_bytes);

// One bound parameter: the model role, its layer and the archive tensor.
struct Binding {
  int role;
  uint32_t layer;
  const dl::archive::Tensor* tensor;
};

// Serialized name of a role (checkpoint.cpp:113-149).
std::string tensor_name(int role, uint32_t layer);

// bind_parameters (checkpoint.cpp:289-318): exactly the 3 + 11 L tensors of
// the config, each with its dense shape and the weight type.
std::vector<Binding> bind_parameters(const Settings& settings, const std::vector<dl::archive::Tensor>& catalog);

// bind_causal_lm (checkpoint.cpp:345-360): the config artifact parsed with
// the first catalog tensor's type, then the parameter binding.
Settings bind_causal_lm(const dl_archive& archive, std::string_view configuration_artifact,
                        std::vector<Binding>* bindings);

}  // namespace dl::qwen3
