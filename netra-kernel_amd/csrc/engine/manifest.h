// Host-only model of an engine directory's engine.json (format netra-engine-1).
// Parsing and validation live here, free of HIP calls, so that the manifest
// contract is testable without a GPU.
//
// Fields read follow the reference runtime's reader
// (runtime/gfx950/engine/netra_engine.hip:273-383): format_version, target,
// wave_size, required_rocm{minimum, code_object_version}, workspace_bytes,
// profiles[].guards{m,batch,sequence}{min,max}, profiles[].tensor_parallel,
// operations[]{execution, launch{grid,block,lds_bytes,dynamic_lds_bytes},
// hsaco, kernel_symbol, arguments[]{kind, source, workspace_offset, value}}.
#pragma once

#include <array>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace netra {

constexpr uint32_t kMaxArguments = 32;

// Minimal JSON document: objects, arrays, strings, numbers, bools, null.
struct JsonValue {
  enum class Type { Null, Bool, Number, String, Array, Object };
  Type type = Type::Null;
  bool boolean = false;
  bool is_unsigned = false;  // number was a plain non-negative integer
  uint64_t unsigned_value = 0;
  double number = 0.0;
  std::string text;
  std::vector<JsonValue> items;
  std::vector<std::pair<std::string, JsonValue>> members;

  const JsonValue* get(const std::string& key) const;
  const JsonValue& require(const std::string& key) const;
};

JsonValue parse_json(const std::string& source);  // throws std::runtime_error

struct ArgumentSpec {
  enum class Kind { Binding, Workspace, U32 };
  Kind kind = Kind::Binding;
  uint64_t workspace_offset = 0;
  uint32_t value = 0;
};

struct OperationSpec {
  std::string name;
  bool fallback = true;
  std::array<uint32_t, 3> grid{1, 1, 1};
  std::array<uint32_t, 3> block{1, 1, 1};
  uint32_t lds_bytes = 0;
  uint32_t dynamic_lds_bytes = 0;
  std::string hsaco;  // engine-relative, normalised "hsaco/..."
  std::string kernel_symbol;
  std::vector<ArgumentSpec> arguments;
};

struct ProfileSpec {
  std::string name;
  uint32_t min_m = 0, max_m = 0, min_batch = 0, max_batch = 0;
  uint64_t min_sequence = 0, max_sequence = 0;
  uint32_t tensor_parallel = 1;
};

struct EngineManifest {
  uint32_t rocm_major = 0, rocm_minor = 0;
  uint64_t workspace_bytes = 0;
  std::vector<ProfileSpec> profiles;
  std::vector<OperationSpec> operations;
};

// Reads and validates <directory>/engine.json. Throws std::runtime_error with
// a human-readable reason on any contract violation.
EngineManifest load_manifest(const std::string& directory);

// "hsaco/<components>" with no empty, "." or ".." component and no backslash.
bool is_normalised_hsaco_path(const std::string& relative);

}  // namespace netra
