// Host-only engine.json reader and validator (no HIP calls).
#include "manifest.h"

#include <cctype>
#include <cstdlib>
#include <fstream>
#include <limits>
#include <sstream>

namespace netra {

const JsonValue* JsonValue::get(const std::string& key) const {
  if (type != Type::Object) return nullptr;
  for (const auto& m : members)
    if (m.first == key) return &m.second;
  return nullptr;
}

const JsonValue& JsonValue::require(const std::string& key) const {
  const JsonValue* v = get(key);
  if (!v) throw std::runtime_error("engine.json: missing field '" + key + "'");
  return *v;
}

namespace {

class Reader {
 public:
  explicit Reader(const std::string& s) : s_(s) {}

  JsonValue document() {
    JsonValue v = value(0);
    skip();
    if (i_ != s_.size()) error("unexpected trailing characters");
    return v;
  }

 private:
  const std::string& s_;
  size_t i_ = 0;

  [[noreturn]] void error(const std::string& what) const {
    throw std::runtime_error("engine.json: " + what + " (offset " + std::to_string(i_) + ")");
  }
  void skip() {
    while (i_ < s_.size() && std::isspace(static_cast<unsigned char>(s_[i_]))) ++i_;
  }
  bool take(char c) {
    skip();
    if (i_ < s_.size() && s_[i_] == c) { ++i_; return true; }
    return false;
  }
  bool literal(const char* word) {
    const size_t n = std::char_traits<char>::length(word);
    if (s_.compare(i_, n, word) == 0) { i_ += n; return true; }
    return false;
  }

  JsonValue value(int depth) {
    if (depth > 64) error("nesting too deep");
    skip();
    if (i_ >= s_.size()) error("unexpected end of input");
    JsonValue v;
    const char c = s_[i_];
    if (c == '{') {
      ++i_;
      v.type = JsonValue::Type::Object;
      if (take('}')) return v;
      do {
        skip();
        if (i_ >= s_.size() || s_[i_] != '"') error("expected a member name");
        std::string key = string();
        for (const auto& m : v.members)
          if (m.first == key) error("duplicate member '" + key + "'");
        if (!take(':')) error("expected ':'");
        v.members.emplace_back(std::move(key), value(depth + 1));
      } while (take(','));
      if (!take('}')) error("expected '}'");
    } else if (c == '[') {
      ++i_;
      v.type = JsonValue::Type::Array;
      if (take(']')) return v;
      do { v.items.push_back(value(depth + 1)); } while (take(','));
      if (!take(']')) error("expected ']'");
    } else if (c == '"') {
      v.type = JsonValue::Type::String;
      v.text = string();
    } else if (c == '-' || (c >= '0' && c <= '9')) {
      number(v);
    } else if (literal("true")) {
      v.type = JsonValue::Type::Bool; v.boolean = true;
    } else if (literal("false")) {
      v.type = JsonValue::Type::Bool;
    } else if (literal("null")) {
      v.type = JsonValue::Type::Null;
    } else {
      error("unexpected character");
    }
    return v;
  }

  std::string string() {
    ++i_;  // opening quote
    std::string out;
    while (i_ < s_.size()) {
      const char c = s_[i_++];
      if (c == '"') return out;
      if (static_cast<unsigned char>(c) < 0x20) error("control character in string");
      if (c != '\\') { out.push_back(c); continue; }
      if (i_ >= s_.size()) break;
      const char esc = s_[i_++];
      switch (esc) {
        case '"': case '\\': case '/': out.push_back(esc); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        case 'u': {
          if (i_ + 4 > s_.size()) error("short \\u escape");
          const unsigned long cp = std::strtoul(s_.substr(i_, 4).c_str(), nullptr, 16);
          i_ += 4;
          if (cp < 0x80) out.push_back(static_cast<char>(cp));
          else error("non-ASCII \\u escapes are not supported");
          break;
        }
        default: error("bad escape");
      }
    }
    error("unterminated string");
  }

  void number(JsonValue& v) {
    const size_t start = i_;
    bool integral = true, negative = false;
    if (s_[i_] == '-') { negative = true; ++i_; }
    while (i_ < s_.size() && std::isdigit(static_cast<unsigned char>(s_[i_]))) ++i_;
    if (i_ < s_.size() && (s_[i_] == '.' || s_[i_] == 'e' || s_[i_] == 'E')) {
      integral = false;
      ++i_;
      while (i_ < s_.size() && (std::isdigit(static_cast<unsigned char>(s_[i_])) ||
                                s_[i_] == '+' || s_[i_] == '-' || s_[i_] == 'e' || s_[i_] == 'E'))
        ++i_;
    }
    const std::string token = s_.substr(start, i_ - start);
    if (token == "-" || token.empty()) error("bad number");
    v.type = JsonValue::Type::Number;
    v.number = std::strtod(token.c_str(), nullptr);
    if (integral && !negative) {
      uint64_t acc = 0;
      for (char d : token) {
        const uint64_t digit = static_cast<uint64_t>(d - '0');
        if (acc > (std::numeric_limits<uint64_t>::max() - digit) / 10) error("integer overflow");
        acc = acc * 10 + digit;
      }
      v.is_unsigned = true;
      v.unsigned_value = acc;
    }
  }
};

uint64_t as_u64(const JsonValue& v, const char* what) {
  if (v.type != JsonValue::Type::Number || !v.is_unsigned)
    throw std::runtime_error(std::string("engine.json: ") + what + " must be a non-negative integer");
  return v.unsigned_value;
}

uint32_t as_u32(const JsonValue& v, const char* what) {
  const uint64_t x = as_u64(v, what);
  if (x > std::numeric_limits<uint32_t>::max())
    throw std::runtime_error(std::string("engine.json: ") + what + " exceeds uint32");
  return static_cast<uint32_t>(x);
}

const std::string& as_text(const JsonValue& v, const char* what) {
  if (v.type != JsonValue::Type::String)
    throw std::runtime_error(std::string("engine.json: ") + what + " must be a string");
  return v.text;
}

void parse_rocm_version(const std::string& text, uint32_t& major, uint32_t& minor) {
  const size_t dot = text.find('.');
  const bool ok = dot != std::string::npos && dot > 0 && dot + 1 < text.size() &&
                  text.find('.', dot + 1) == std::string::npos;
  if (ok) {
    for (size_t i = 0; i < text.size(); ++i)
      if (i != dot && !std::isdigit(static_cast<unsigned char>(text[i])))
        throw std::runtime_error("engine.json: required_rocm.minimum must be MAJOR.MINOR");
    const unsigned long long a = std::strtoull(text.substr(0, dot).c_str(), nullptr, 10);
    const unsigned long long b = std::strtoull(text.substr(dot + 1).c_str(), nullptr, 10);
    if (a > 0xffffffffull || b > 0xffffffffull)
      throw std::runtime_error("engine.json: required_rocm.minimum overflows uint32");
    major = static_cast<uint32_t>(a);
    minor = static_cast<uint32_t>(b);
    return;
  }
  throw std::runtime_error("engine.json: required_rocm.minimum must be MAJOR.MINOR");
}

void read_range32(const JsonValue& guards, const char* name, uint32_t& lo, uint32_t& hi) {
  const JsonValue& g = guards.require(name);
  lo = as_u32(g.require("min"), name);
  hi = as_u32(g.require("max"), name);
  if (lo > hi) throw std::runtime_error(std::string("engine.json: guard ") + name + " has min > max");
}

}  // namespace

JsonValue parse_json(const std::string& source) { return Reader(source).document(); }

bool is_normalised_hsaco_path(const std::string& p) {
  if (p.size() <= 6 || p.compare(0, 6, "hsaco/") != 0) return false;
  if (p.find('\\') != std::string::npos) return false;
  size_t start = 0;
  while (start <= p.size()) {
    size_t end = p.find('/', start);
    if (end == std::string::npos) end = p.size();
    const std::string part = p.substr(start, end - start);
    if (part.empty() || part == "." || part == "..") return false;
    start = end + 1;
    if (end == p.size()) break;
  }
  return true;
}

EngineManifest load_manifest(const std::string& directory) {
  const std::string path = directory + "/engine.json";
  std::ifstream in(path, std::ios::binary);
  if (!in) throw std::runtime_error("cannot open " + path);
  std::stringstream buffer;
  buffer << in.rdbuf();
  const JsonValue root = parse_json(buffer.str());
  if (root.type != JsonValue::Type::Object) throw std::runtime_error("engine.json: root must be an object");

  if (as_text(root.require("format_version"), "format_version") != "netra-engine-1")
    throw std::runtime_error("engine.json: format_version must be netra-engine-1");
  if (as_text(root.require("target"), "target") != "gfx950")
    throw std::runtime_error("engine.json: target must be gfx950");
  if (as_u32(root.require("wave_size"), "wave_size") != 64)
    throw std::runtime_error("engine.json: wave_size must be 64");

  EngineManifest m;
  const JsonValue& rocm = root.require("required_rocm");
  if (as_u32(rocm.require("code_object_version"), "code_object_version") != 6)
    throw std::runtime_error("engine.json: only code object version 6 is supported");
  parse_rocm_version(as_text(rocm.require("minimum"), "required_rocm.minimum"), m.rocm_major,
                     m.rocm_minor);
  m.workspace_bytes = as_u64(root.require("workspace_bytes"), "workspace_bytes");

  const JsonValue& profiles = root.require("profiles");
  const JsonValue& operations = root.require("operations");
  if (profiles.type != JsonValue::Type::Array || operations.type != JsonValue::Type::Array)
    throw std::runtime_error("engine.json: profiles and operations must be arrays");

  for (const JsonValue& p : profiles.items) {
    ProfileSpec spec;
    if (const JsonValue* n = p.get("name")) spec.name = as_text(*n, "profile.name");
    const JsonValue& guards = p.require("guards");
    read_range32(guards, "m", spec.min_m, spec.max_m);
    read_range32(guards, "batch", spec.min_batch, spec.max_batch);
    const JsonValue& seq = guards.require("sequence");
    spec.min_sequence = as_u64(seq.require("min"), "sequence.min");
    spec.max_sequence = as_u64(seq.require("max"), "sequence.max");
    if (spec.min_sequence > spec.max_sequence)
      throw std::runtime_error("engine.json: guard sequence has min > max");
    spec.tensor_parallel = as_u32(p.require("tensor_parallel"), "tensor_parallel");
    m.profiles.push_back(spec);
  }

  for (const JsonValue& o : operations.items) {
    OperationSpec op;
    if (const JsonValue* n = o.get("name")) op.name = as_text(*n, "operation.name");
    op.fallback = as_text(o.require("execution"), "execution") != "kernel";
    if (const JsonValue* launch = o.get("launch"); launch && launch->type == JsonValue::Type::Object) {
      const JsonValue& grid = launch->require("grid");
      const JsonValue& block = launch->require("block");
      if (grid.type != JsonValue::Type::Array || grid.items.size() != 3 ||
          block.type != JsonValue::Type::Array || block.items.size() != 3)
        throw std::runtime_error("engine.json: launch grid and block need three dimensions");
      for (int d = 0; d < 3; ++d) {
        op.grid[d] = as_u32(grid.items[d], "grid");
        op.block[d] = as_u32(block.items[d], "block");
        if (op.grid[d] == 0 || op.block[d] == 0)
          throw std::runtime_error("engine.json: launch dimensions must be nonzero");
      }
      if (static_cast<uint64_t>(op.block[0]) * op.block[1] * op.block[2] > 1024)
        throw std::runtime_error("engine.json: workgroup larger than 1024 threads");
      op.lds_bytes = as_u32(launch->require("lds_bytes"), "lds_bytes");
      if (const JsonValue* d = launch->get("dynamic_lds_bytes"))
        op.dynamic_lds_bytes = as_u32(*d, "dynamic_lds_bytes");
      if (static_cast<uint64_t>(op.lds_bytes) + op.dynamic_lds_bytes > 160u * 1024u)
        throw std::runtime_error("engine.json: LDS request exceeds 160 KiB");
    }
    if (!op.fallback) {
      if (!o.get("launch")) throw std::runtime_error("engine.json: kernel operation without launch");
      op.hsaco = as_text(o.require("hsaco"), "hsaco");
      if (!is_normalised_hsaco_path(op.hsaco))
        throw std::runtime_error("engine.json: hsaco must be a normalised hsaco/... path");
      op.kernel_symbol = as_text(o.require("kernel_symbol"), "kernel_symbol");
      if (op.kernel_symbol.empty()) throw std::runtime_error("engine.json: empty kernel_symbol");
      const JsonValue& args = o.require("arguments");
      if (args.type != JsonValue::Type::Array || args.items.empty())
        throw std::runtime_error("engine.json: kernel operation needs typed arguments");
      if (args.items.size() > kMaxArguments)
        throw std::runtime_error("engine.json: more than 32 kernel arguments");
      for (const JsonValue& a : args.items) {
        ArgumentSpec arg;
        const std::string& kind = as_text(a.require("kind"), "argument.kind");
        if (kind == "pointer") {
          std::string source = "binding";
          if (const JsonValue* s = a.get("source")) source = as_text(*s, "argument.source");
          if (source == "binding") {
            arg.kind = ArgumentSpec::Kind::Binding;
          } else if (source == "workspace") {
            arg.kind = ArgumentSpec::Kind::Workspace;
            arg.workspace_offset = as_u64(a.require("workspace_offset"), "workspace_offset");
            if (arg.workspace_offset >= m.workspace_bytes)
              throw std::runtime_error("engine.json: workspace_offset outside the workspace");
          } else {
            throw std::runtime_error("engine.json: unsupported pointer source '" + source + "'");
          }
        } else if (kind == "u32_constant") {
          arg.kind = ArgumentSpec::Kind::U32;
          arg.value = as_u32(a.require("value"), "argument.value");
        } else {
          throw std::runtime_error("engine.json: unsupported argument kind '" + kind + "'");
        }
        op.arguments.push_back(arg);
      }
    }
    m.operations.push_back(std::move(op));
  }
  return m;
}

}  // namespace netra
